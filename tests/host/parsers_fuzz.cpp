// Host-side robustness check of the weight-pack reader, the JSON parser and
// the model-config parser, meant to be built with AddressSanitizer and
// UndefinedBehaviorSanitizer (tests/test_host_sanitize.py). The reference
// runs its suites under compute-sanitizer (tests/run_sanitizers.sh); GPU
// sanitizers are not available on the target pool, so the host code that
// parses untrusted files is checked here instead.
//
// A valid OPWPACK1 pack is built in memory, checked to load and read back
// exactly, then mutated deterministically (byte flips, truncation, inserted
// bytes, numbers replaced by extreme literals) a few thousand times. Every
// mutant must either load and read in bounds or throw std::exception; any
// memory error or undefined behaviour aborts the process under the
// sanitizers. Usage: parsers_fuzz <scratch directory> [iterations]

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "json.hpp"
#include "model_config.hpp"
#include "pack_reader.hpp"

using opworks::ModelConfig;
using opworks::PackReader;

namespace {

uint64_t g_state = 0x9E3779B97F4A7C15ull;
uint64_t next_u64() { // xorshift64*
    g_state ^= g_state >> 12;
    g_state ^= g_state << 25;
    g_state ^= g_state >> 27;
    return g_state * 0x2545F4914F6CDD1Dull;
}
size_t below(size_t n) { return n ? static_cast<size_t>(next_u64() % n) : 0; }

const char *kManifest = R"({"format_version": 1, "dtype": "float32",
 "config": {"num_hidden_layers": 2, "hidden_size": 8, "intermediate_size": 16, "num_attention_heads": 2,
            "num_key_value_heads": 1, "head_dim": 4, "vocab_size": 12, "rms_norm_eps": 1e-5,
            "rope_theta": 500000.0, "rope_scaling": {"rope_type": "llama3", "factor": 32.0,
            "low_freq_factor": 1.0, "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}},
 "eos_token_ids": [3, 5],
 "tensors": {"embed": {"offset": 0, "shape": [12, 8]}, "norm": {"offset": 384, "shape": [8]},
             "w\u00e9\ud83d\ude00": {"offset": 448, "shape": [2, 2]}},
 "aliases": {"lm_head": "embed"}})";

std::string make_pack(const std::string &manifest, size_t blob_bytes) {
    std::string out("OPWPACK1");
    uint64_t n = manifest.size();
    for (int i = 0; i < 8; ++i)
        out += static_cast<char>((n >> (8 * i)) & 0xFF);
    out += manifest;
    for (size_t i = 0; i < blob_bytes; ++i)
        out += static_cast<char>(i * 7 + 1);
    return out;
}

void write_file(const std::string &path, const std::string &bytes) {
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(bytes.data(), 1, bytes.size(), f) != bytes.size()) {
        std::fprintf(stderr, "cannot write %s\n", path.c_str());
        std::exit(2);
    }
    std::fclose(f);
}

// Loads a pack the way the model loader does; returns true if it was accepted.
bool exercise(const std::string &path) {
    try {
        PackReader r(path);
        (void)ModelConfig::from_manifest(r.manifest());
        for (const auto &[name, meta] : r.manifest().at("tensors").as_object()) {
            (void)meta;
            const PackReader::TensorMeta &m = r.meta(name);
            std::vector<unsigned char> buf(static_cast<size_t>(m.numel) * r.elem_size());
            r.read_into(name, buf.data(), buf.size());
        }
        if (r.has("lm_head"))
            (void)r.meta("lm_head");
        return true;
    } catch (const std::exception &) {
        return false;
    }
}

bool json_accepts(const std::string &text) {
    try {
        opworks::json::Value v = opworks::json::parse(text);
        if (v.is_object())
            (void)ModelConfig::from_json(v, v.find("eos"));
        return true;
    } catch (const std::exception &) {
        return false;
    }
}

int g_fail = 0;
void expect(bool ok, const char *what) {
    if (!ok) {
        std::fprintf(stderr, "FAIL: %s\n", what);
        ++g_fail;
    }
}

std::string mutate(std::string s) {
    static const char *kLiterals[] = {"1e999", "-1", "-0", "9223372036854775807", "18446744073709551616",
                                      "4294967296", "2147483648", "0.5", "nan", "\"x\"", "[]", "{}", "null",
                                      "-9007199254740993", "1e-400"};
    const int kind = static_cast<int>(below(6));
    if (s.empty())
        return s;
    if (kind == 0) { // flip bytes
        for (int i = 0, n = 1 + static_cast<int>(below(4)); i < n; ++i)
            s[below(s.size())] ^= static_cast<char>(1u << below(8));
    } else if (kind == 1) { // truncate
        s.resize(below(s.size()));
    } else if (kind == 2) { // insert random bytes
        std::string ins;
        for (int i = 0, n = 1 + static_cast<int>(below(8)); i < n; ++i)
            ins += static_cast<char>(below(256));
        s.insert(below(s.size()), ins);
    } else if (kind == 3) { // replace a run of digits with an extreme literal
        size_t p = s.find_first_of("0123456789", below(s.size()));
        if (p != std::string::npos) {
            size_t q = s.find_first_not_of("0123456789.e-", p);
            s.replace(p, (q == std::string::npos ? s.size() : q) - p, kLiterals[below(15)]);
        }
    } else if (kind == 4) { // delete a span
        size_t p = below(s.size());
        s.erase(p, below(16));
    } else { // duplicate a span
        size_t p = below(s.size());
        s.insert(below(s.size()), s.substr(p, below(32)));
    }
    return s;
}

} // namespace

int main(int argc, char **argv) {
    if (argc < 2) {
        std::fprintf(stderr, "usage: %s <scratch dir> [iterations]\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    const int iters = argc > 2 ? std::atoi(argv[2]) : 3000;
    const std::string path = dir + "/fuzz.pack";
    const size_t blob = 464;

    // known answer: the valid pack loads and reads its bytes back exactly
    const std::string good = make_pack(kManifest, blob);
    write_file(path, good);
    {
        PackReader r(path);
        ModelConfig c = ModelConfig::from_manifest(r.manifest());
        expect(c.num_layers == 2 && c.hidden_size == 8 && c.eos_token_ids.size() == 2, "config fields");
        expect(r.has("lm_head") && r.meta("lm_head").numel == 96, "alias resolves");
        std::vector<unsigned char> norm(32);
        r.read_into("norm", norm.data(), norm.size());
        for (size_t i = 0; i < norm.size(); ++i)
            expect(norm[i] == static_cast<unsigned char>((384 + i) * 7 + 1), "norm bytes");
        expect(r.manifest().at("tensors").find("w\xc3\xa9\xf0\x9f\x98\x80") != nullptr, "utf-8 escapes");
        bool small_dst = false;
        try {
            r.read_into("norm", norm.data(), 31);
        } catch (const std::exception &) {
            small_dst = true;
        }
        expect(small_dst, "short destination rejected");
    }

    // hand-picked malformed manifests that must be rejected
    auto manifest_with = [](const std::string &from, const std::string &to) {
        std::string m(kManifest);
        size_t p = m.find(from);
        if (p == std::string::npos) {
            std::fprintf(stderr, "bad case %s\n", from.c_str());
            std::exit(2);
        }
        return m.replace(p, from.size(), to);
    };
    const std::pair<const char *, const char *> bad[] = {
        {"\"offset\": 384", "\"offset\": -8"},
        {"\"offset\": 384", "\"offset\": 18446744073709551608"},
        {"\"offset\": 384", "\"offset\": 1e999"},
        {"\"shape\": [8]", "\"shape\": [4294967296, 4294967296]"},
        {"\"shape\": [8]", "\"shape\": [0]"},
        {"\"shape\": [8]", "\"shape\": [30]"},
        {"\"hidden_size\": 8", "\"hidden_size\": 4294967304"},
        {"\"hidden_size\": 8", "\"hidden_size\": 8.5"},
        {"\"head_dim\": 4", "\"head_dim\": 1073741824"},
        {"\"rms_norm_eps\": 1e-5", "\"rms_norm_eps\": 1e300"},
        {"\"eos_token_ids\": [3, 5]", "\"eos_token_ids\": [3, 1e20]"},
        {"\"format_version\": 1", "\"format_version\": 2"},
        {"\"dtype\": \"float32\"", "\"dtype\": \"int8\""},
        {"\"lm_head\": \"embed\"", "\"lm_head\": \"missing\""},
        {"\"rope_type\": \"llama3\"", "\"rope_type\": \"yarn\""},
    };
    for (const auto &[from, to] : bad) {
        write_file(path, make_pack(manifest_with(from, to), blob));
        if (exercise(path)) {
            std::fprintf(stderr, "accepted: %s\n", to);
            ++g_fail;
        }
    }
    const char *bad_json[] = {"", "{", "[1,", "\"\\u12\"", "\"\\ud800\\u0041\"", "{\"a\" 1}", "01x", "-",
                              "[1] 2", "\"\x01\"", "tru", "{\"a\":}", "1e", "\"\\q\""};
    for (const char *j : bad_json)
        expect(!json_accepts(j), j);
    expect(json_accepts("{\"a\": [1, 2.5e3, -0, true, null, \"\\u00e9\"]}") == false, "object without config keys");
    expect(!json_accepts(std::string(300, '[') + std::string(300, ']')), "nesting limit");
    expect(opworks::json::parse(std::string(200, '[') + std::string(200, ']')).is_array(), "nesting within limit");

    // truncated headers
    for (size_t n : {0, 4, 8, 12, 16, 20})
        write_file(path, good.substr(0, n)), expect(!exercise(path), "truncated header");

    // mutation sweep over the whole file and over the manifest alone
    int accepted = 0;
    for (int it = 0; it < iters; ++it) {
        std::string mutant = (it & 1) ? mutate(good) : make_pack(mutate(kManifest), blob);
        write_file(path, mutant);
        accepted += exercise(path);
        (void)json_accepts(mutate(kManifest));
    }
    std::printf("parsers_fuzz: %d iterations, %d mutants accepted, %d failures\n", iters, accepted, g_fail);
    return g_fail ? 1 : 0;
}

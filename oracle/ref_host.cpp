// Test-only C shim over the reference's own host code, compiled in place from
// /root/reference/include/runtime/{json,model_config,pack_reader}.cuh (plain
// C++17, no CUDA) by oracle/ref_host.mk into oracle/_ref/. It lets tests check
// this build's RoPE frequencies and pack handling against the reference's
// implementation itself. Nothing in the product links it.
#include <cstdint>
#include <cstring>
#include <string>

#include "runtime/model_config.cuh"
#include "runtime/pack_reader.cuh"

extern "C" {

// ModelConfig::from_manifest(manifest).rope_inv_freq() into out (n floats). 0 / -1.
int ref_rope_inv_freq(const char *manifest_json, float *out, int n) {
    try {
        opworks::ModelConfig c = opworks::ModelConfig::from_manifest(opworks::json::parse(manifest_json));
        std::vector<float> f = c.rope_inv_freq();
        if (static_cast<int>(f.size()) != n)
            return -1;
        std::memcpy(out, f.data(), sizeof(float) * f.size());
        return 0;
    } catch (...) {
        return -1;
    }
}

// PackReader(path).read(name) for a float32 pack, into out (n floats). Returns numel or -1.
int64_t ref_pack_read_f32(const char *path, const char *name, float *out, int64_t n) {
    try {
        opworks::PackReader p(path);
        std::vector<float> v = p.read(name);
        if (static_cast<int64_t>(v.size()) > n)
            return -1;
        std::memcpy(out, v.data(), sizeof(float) * v.size());
        return static_cast<int64_t>(v.size());
    } catch (...) {
        return -1;
    }
}

} // extern "C"

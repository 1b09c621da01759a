#pragma once

// Reader of OpWorks weight packs, format "OPWPACK1" (reference writer:
// scripts/llama/pack_format.py:1-17, 59-87; reader: include/runtime/pack_reader.cuh):
//   [8 B magic "OPWPACK1"][u64 LE manifest length][JSON manifest][blob]
// The manifest holds format_version 1, dtype "float32" | "bfloat16", tensors
// {name: {offset (bytes into the blob, 64-B aligned), shape}}, optional
// aliases {alias: target}, plus config / eos_token_ids / meta keys. Tensors
// are read straight from the file into caller memory (pinned staging
// buffers), one tensor at a time.

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "json.hpp"

namespace opworks {

class PackReader {
  public:
    struct TensorMeta {
        uint64_t offset = 0; // bytes from the blob start
        std::vector<int64_t> shape;
        int64_t numel = 0;
    };

    explicit PackReader(const std::string &path) : path_(path) {
        FILE *f = std::fopen(path.c_str(), "rb");
        if (!f)
            throw std::runtime_error("cannot open pack " + path);
        struct Closer {
            FILE *f;
            ~Closer() { std::fclose(f); }
        } closer{f};
        char magic[8];
        if (std::fread(magic, 1, 8, f) != 8 || std::memcmp(magic, "OPWPACK1", 8) != 0)
            throw std::runtime_error(path + ": not an OpWorks pack (bad magic)");
        unsigned char lenb[8];
        if (std::fread(lenb, 1, 8, f) != 8)
            throw std::runtime_error(path + ": corrupt manifest length");
        uint64_t json_len = 0;
        for (int i = 7; i >= 0; --i)
            json_len = (json_len << 8) | lenb[i];
        if (json_len > (1ull << 30))
            throw std::runtime_error(path + ": corrupt manifest length");
        std::string js(json_len, '\0');
        if (json_len && std::fread(&js[0], 1, json_len, f) != json_len)
            throw std::runtime_error(path + ": truncated manifest");
        blob_offset_ = 16 + json_len;
        if (std::fseek(f, 0, SEEK_END) != 0)
            throw std::runtime_error(path + ": cannot seek");
        const long end = std::ftell(f);
        if (end < 0 || static_cast<uint64_t>(end) < blob_offset_)
            throw std::runtime_error(path + ": truncated pack");
        blob_size_ = static_cast<uint64_t>(end) - blob_offset_;

        manifest_ = json::parse(js);
        if (manifest_.at("format_version").as_int() != 1)
            throw std::runtime_error(path + ": unsupported format version");
        dtype_ = manifest_.at("dtype").as_string();
        if (dtype_ == "float32")
            elem_size_ = 4;
        else if (dtype_ == "bfloat16")
            elem_size_ = 2;
        else
            throw std::runtime_error(path + ": unsupported dtype " + dtype_);
        for (const auto &[name, meta] : manifest_.at("tensors").as_object()) {
            TensorMeta m;
            const int64_t offset = meta.at("offset").as_int();
            if (offset < 0)
                throw std::runtime_error(path + ": negative offset in " + name);
            m.offset = static_cast<uint64_t>(offset);
            m.numel = 1;
            for (const auto &d : meta.at("shape").as_array()) {
                const int64_t dim = d.as_int();
                if (dim <= 0)
                    throw std::runtime_error(path + ": non-positive dim in " + name);
                if (dim > (1ll << 40) / m.numel)
                    throw std::runtime_error(path + ": absurd tensor size in " + name);
                m.numel *= dim;
                m.shape.push_back(dim);
            }
            if (m.offset > blob_size_ || static_cast<uint64_t>(m.numel) * elem_size_ > blob_size_ - m.offset)
                throw std::runtime_error(path + ": tensor " + name + " overruns the data blob");
            tensors_.emplace(name, std::move(m));
        }
        if (const json::Value *aliases = manifest_.find("aliases")) {
            for (const auto &[alias, target] : aliases->as_object()) {
                if (!tensors_.count(target.as_string()))
                    throw std::runtime_error(path + ": alias " + alias + " targets missing tensor " +
                                             target.as_string());
                aliases_.emplace(alias, target.as_string());
            }
        }
    }

    const std::string &path() const { return path_; }
    const std::string &dtype() const { return dtype_; }
    size_t elem_size() const { return elem_size_; }
    const json::Value &manifest() const { return manifest_; }

    bool has(const std::string &name) const { return tensors_.count(name) || aliases_.count(name); }

    const TensorMeta &meta(const std::string &name) const {
        auto a = aliases_.find(name);
        const std::string &key = a == aliases_.end() ? name : a->second;
        auto it = tensors_.find(key);
        if (it == tensors_.end())
            throw std::runtime_error(path_ + ": missing tensor " + name);
        return it->second;
    }

    // Copies one tensor's bytes (numel * elem_size) into dst.
    void read_into(const std::string &name, void *dst, size_t dst_bytes) const {
        const TensorMeta &m = meta(name);
        const size_t bytes = static_cast<size_t>(m.numel) * elem_size_;
        if (dst_bytes < bytes)
            throw std::runtime_error(path_ + ": destination too small for " + name);
        FILE *f = std::fopen(path_.c_str(), "rb");
        if (!f)
            throw std::runtime_error("cannot reopen pack " + path_);
        const bool ok = std::fseek(f, static_cast<long>(blob_offset_ + m.offset), SEEK_SET) == 0 &&
                        std::fread(dst, 1, bytes, f) == bytes;
        std::fclose(f);
        if (!ok)
            throw std::runtime_error(path_ + ": failed reading tensor " + name);
    }

    // Host-vector readers (interface of the reference's PackReader,
    // include/runtime/pack_reader.cuh:109-160), all built on read_into.

    // One tensor's bytes as stored.
    std::vector<uint8_t> read_raw(const std::string &name) const {
        std::vector<uint8_t> out(static_cast<size_t>(meta(name).numel) * elem_size_);
        read_into(name, out.data(), out.size());
        return out;
    }

    // A tensor of a float32 pack.
    std::vector<float> read(const std::string &name) const {
        if (dtype_ != "float32")
            throw std::runtime_error(path_ + ": read() requires a float32 pack; use read_raw for " + dtype_);
        std::vector<float> out(static_cast<size_t>(meta(name).numel));
        read_into(name, out.data(), out.size() * sizeof(float));
        return out;
    }

    // A tensor of a bfloat16 pack, each value widened exactly to fp32.
    std::vector<float> read_bf16_as_float(const std::string &name) const {
        if (dtype_ != "bfloat16")
            throw std::runtime_error(path_ + ": read_bf16_as_float requires a bfloat16 pack");
        std::vector<uint16_t> bits(static_cast<size_t>(meta(name).numel));
        read_into(name, bits.data(), bits.size() * sizeof(uint16_t));
        std::vector<float> out(bits.size());
        for (size_t i = 0; i < bits.size(); ++i) {
            const uint32_t word = static_cast<uint32_t>(bits[i]) << 16;
            std::memcpy(&out[i], &word, sizeof(word));
        }
        return out;
    }

    // int32 values stored bit for bit in a float32 tensor (how fixture packs
    // carry token ids; model packs hold no such tensor).
    std::vector<int32_t> read_int32(const std::string &name) const {
        if (dtype_ != "float32")
            throw std::runtime_error(path_ + ": read_int32 requires a float32 pack");
        std::vector<int32_t> out(static_cast<size_t>(meta(name).numel));
        read_into(name, out.data(), out.size() * sizeof(int32_t));
        return out;
    }

  private:
    std::string path_, dtype_;
    size_t elem_size_ = 4;
    json::Value manifest_;
    std::map<std::string, TensorMeta> tensors_;
    std::map<std::string, std::string> aliases_;
    uint64_t blob_offset_ = 0, blob_size_ = 0;
};

} // namespace opworks

#pragma once

// Reader of OpWorks weight packs, file format "OPWPACK1" (written by the
// reference's scripts/llama/pack_format.py:1-17, 59-87):
//   [8 B magic "OPWPACK1"][u64 little-endian manifest length][JSON manifest][blob]
// The manifest holds format_version 1, dtype "float32" | "bfloat16", tensors
// {name: {offset (bytes into the blob), shape}}, optional aliases
// {alias: target}, plus config / eos_token_ids / meta keys.
//
// The public surface is the reference's PackReader (has, meta, dtype,
// elem_size, manifest, read_raw, read, read_bf16_as_float, read_int32;
// include/runtime/pack_reader.cuh:17-175), plus read_into (copy into caller
// memory, e.g. a pinned staging buffer) and bytes (a zero-copy view).
//
// How it reads: the file is mapped read-only once for the reader's lifetime
// (shared by copies of the reader) and everything is parsed out of the mapping.
// One pass over the manifest builds a table of entries, each tensor's byte
// range proven to lie inside the blob with overflow-checked arithmetic, and
// aliases are resolved into the same name index at that time, so a lookup is
// one map probe and a read is a memcpy out of the mapping: no file is reopened
// and nothing is seeked per tensor. The only size limits are the file's own:
// the manifest must fit in the file and every tensor in the blob.

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
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

    explicit PackReader(const std::string &path) : path_(path), file_(map_file(path)) {
        const uint8_t *p = file_->data;
        const uint64_t size = file_->size;
        static constexpr char kMagic[8] = {'O', 'P', 'W', 'P', 'A', 'C', 'K', '1'};
        if (size < sizeof(kMagic) || std::memcmp(p, kMagic, sizeof(kMagic)) != 0)
            fail("is not an OPWPACK1 file (magic bytes differ)");
        if (size < 16)
            fail("ends inside its 16-byte header");
        uint64_t manifest_bytes = 0;
        for (int i = 0; i < 8; ++i) // little-endian, whatever the host's byte order
            manifest_bytes |= uint64_t(p[8 + i]) << (8 * i);
        if (manifest_bytes > size - 16)
            fail("declares a " + std::to_string(manifest_bytes) + "-byte manifest but only " +
                 std::to_string(size - 16) + " bytes follow the header");
        blob_ = p + 16 + manifest_bytes;
        blob_bytes_ = size - 16 - manifest_bytes;
        manifest_ = json::parse(std::string(reinterpret_cast<const char *>(p + 16), manifest_bytes));
        index_manifest();
    }

    const std::string &path() const { return path_; }
    const std::string &dtype() const { return dtype_; }
    size_t elem_size() const { return elem_size_; }
    const json::Value &manifest() const { return manifest_; }

    // True for a tensor name or an alias of one.
    bool has(const std::string &name) const { return by_name_.count(name) != 0; }

    // Shape and blob offset of a tensor (an alias gives its target's).
    const TensorMeta &meta(const std::string &name) const { return entries_[lookup(name)].meta; }

    // A tensor's stored bytes, read in place: valid while any copy of this reader lives.
    std::pair<const void *, size_t> bytes(const std::string &name) const {
        const Entry &e = entries_[lookup(name)];
        return {blob_ + e.meta.offset, e.bytes};
    }

    // Copies a tensor's stored bytes (numel * elem_size) into dst.
    void read_into(const std::string &name, void *dst, size_t dst_bytes) const {
        const auto [src, n] = bytes(name);
        if (dst_bytes < n)
            throw std::runtime_error(path_ + ": tensor " + name + " needs " + std::to_string(n) +
                                     " bytes, the destination holds " + std::to_string(dst_bytes));
        std::memcpy(dst, src, n);
    }

    // One tensor's bytes as stored.
    std::vector<uint8_t> read_raw(const std::string &name) const {
        const auto [src, n] = bytes(name);
        const uint8_t *b = static_cast<const uint8_t *>(src);
        return std::vector<uint8_t>(b, b + n);
    }

    // A tensor of a float32 pack.
    std::vector<float> read(const std::string &name) const {
        require_dtype("float32", "read");
        return copy_as<float>(name);
    }

    // A tensor of a bfloat16 pack, every value widened exactly to fp32 (bits << 16).
    std::vector<float> read_bf16_as_float(const std::string &name) const {
        require_dtype("bfloat16", "read_bf16_as_float");
        const std::vector<uint16_t> bits = copy_as<uint16_t>(name);
        std::vector<float> out(bits.size());
        for (size_t i = 0; i < bits.size(); ++i) {
            const uint32_t word = uint32_t(bits[i]) << 16;
            std::memcpy(&out[i], &word, sizeof(word));
        }
        return out;
    }

    // int32 values stored bit for bit in a float32 tensor (how fixture packs
    // carry token ids; model packs hold no such tensor).
    std::vector<int32_t> read_int32(const std::string &name) const {
        require_dtype("float32", "read_int32");
        return copy_as<int32_t>(name);
    }

  private:
    // The read-only mapping of the whole file, unmapped when the last reader copy goes.
    struct MappedFile {
        const uint8_t *data = nullptr;
        uint64_t size = 0;
        ~MappedFile() {
            if (data && size)
                ::munmap(const_cast<uint8_t *>(data), size);
        }
    };

    struct Entry {
        TensorMeta meta;
        size_t bytes = 0; // numel * elem_size, inside the blob
    };

    static std::shared_ptr<const MappedFile> map_file(const std::string &path) {
        const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0)
            throw std::runtime_error("weight pack " + path + " cannot be opened: " + std::strerror(errno));
        struct stat st {};
        const bool stat_ok = ::fstat(fd, &st) == 0 && S_ISREG(st.st_mode);
        auto file = std::make_shared<MappedFile>();
        if (stat_ok && st.st_size > 0) {
            void *m = ::mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
            if (m != MAP_FAILED) {
                file->data = static_cast<const uint8_t *>(m);
                file->size = static_cast<uint64_t>(st.st_size);
            }
        }
        ::close(fd);
        if (!stat_ok)
            throw std::runtime_error("weight pack " + path + " is not a regular file");
        if (st.st_size > 0 && !file->data)
            throw std::runtime_error("weight pack " + path + " cannot be mapped");
        return file;
    }

    [[noreturn]] void fail(const std::string &what) const { throw std::runtime_error("weight pack " + path_ + " " + what); }

    void require_dtype(const char *want, const char *fn) const {
        if (dtype_ != want)
            throw std::runtime_error(std::string(fn) + " needs a " + want + " pack; " + path_ + " stores " + dtype_);
    }

    size_t lookup(const std::string &name) const {
        const auto it = by_name_.find(name);
        if (it == by_name_.end())
            throw std::runtime_error(path_ + " has no tensor or alias named " + name);
        return it->second;
    }

    template <typename T> std::vector<T> copy_as(const std::string &name) const {
        const auto [src, n] = bytes(name);
        std::vector<T> out(n / sizeof(T));
        std::memcpy(out.data(), src, out.size() * sizeof(T));
        return out;
    }

    // One pass over the manifest: dtype, then every tensor's range, then the aliases.
    void index_manifest() {
        if (manifest_.at("format_version").as_int() != 1)
            fail("has format_version " + std::to_string(manifest_.at("format_version").as_int()) + " (only 1 is read)");
        dtype_ = manifest_.at("dtype").as_string();
        if (dtype_ == "float32")
            elem_size_ = 4;
        else if (dtype_ == "bfloat16")
            elem_size_ = 2;
        else
            fail("stores dtype '" + dtype_ + "' (float32 and bfloat16 are read)");
        for (const auto &[name, desc] : manifest_.at("tensors").as_object()) {
            Entry e;
            const int64_t offset = desc.at("offset").as_int();
            uint64_t bytes = elem_size_;
            int64_t numel = 1;
            for (const json::Value &d : desc.at("shape").as_array()) {
                const int64_t dim = d.as_int();
                if (dim <= 0 || __builtin_mul_overflow(numel, dim, &numel) ||
                    __builtin_mul_overflow(bytes, static_cast<uint64_t>(dim), &bytes))
                    fail("gives tensor " + name + " an empty, negative or overflowing shape");
                e.meta.shape.push_back(dim);
            }
            if (offset < 0 || static_cast<uint64_t>(offset) > blob_bytes_ ||
                bytes > blob_bytes_ - static_cast<uint64_t>(offset))
                fail("places tensor " + name + " (" + std::to_string(bytes) + " bytes at offset " +
                     std::to_string(offset) + ") outside its " + std::to_string(blob_bytes_) + "-byte blob");
            e.meta.offset = static_cast<uint64_t>(offset);
            e.meta.numel = numel;
            e.bytes = static_cast<size_t>(bytes);
            by_name_.emplace(name, entries_.size());
            entries_.push_back(std::move(e));
        }
        if (const json::Value *aliases = manifest_.find("aliases")) {
            // targets are looked up among the tensors alone (no alias of an alias); an alias that
            // reuses a tensor's name refers to its target, as a name lookup resolves aliases first
            std::vector<std::pair<std::string, size_t>> resolved;
            for (const auto &[alias, target] : aliases->as_object()) {
                const auto it = by_name_.find(target.as_string());
                if (it == by_name_.end())
                    fail("aliases " + alias + " to " + target.as_string() + ", which is not a tensor");
                resolved.emplace_back(alias, it->second);
            }
            for (const auto &[alias, index] : resolved)
                by_name_[alias] = index;
        }
    }

    std::string path_;
    std::shared_ptr<const MappedFile> file_;
    const uint8_t *blob_ = nullptr;
    uint64_t blob_bytes_ = 0;
    json::Value manifest_;
    std::string dtype_;
    size_t elem_size_ = 4;
    std::vector<Entry> entries_;
    std::map<std::string, size_t> by_name_; // tensor names and aliases -> entries_ index
};

} // namespace opworks

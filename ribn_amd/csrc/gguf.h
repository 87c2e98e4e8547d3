// GGUF v3 reader over a read-only mapping of the file.
// Semantics follow GgufFile::read_from (crates/gguf/src/lib.rs:199-296):
// magic 0x46554747, version 3 only, bounded strings/arrays/tensor counts,
// duplicate-key rejection, general.alignment (default 32, power of two),
// every tensor offset inside the file, per-type byte_len (:142-168).
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace ribn {

struct GgufValue {
    uint32_t type = 0;     // GGUF value type
    uint64_t u = 0;        // integer / bool payload (sign-extended for signed types)
    double f = 0.0;        // float payload
    std::string s;         // string payload
    uint64_t array_len = 0;
    uint32_t array_type = 0;
    bool is_array = false;
};

struct GgufTensor {
    std::string name;
    std::vector<uint64_t> dims;   // ne0 first
    uint32_t type = 0;
    uint64_t offset = 0;          // relative to the data section
    uint64_t bytes = 0;           // encoded length (0 when the type has no layout here)
};

class GgufFile {
public:
    ~GgufFile();
    // Returns an empty string on success, otherwise the error message.
    std::string open(const std::string& path);
    const GgufValue* get(const std::string& key) const;
    bool get_u64(const std::string& key, uint64_t* out) const;
    bool get_f32(const std::string& key, float* out) const;
    bool get_str(const std::string& key, std::string* out) const;
    const GgufTensor* tensor(const std::string& name) const;
    const uint8_t* data(const GgufTensor& t) const { return base_ + data_offset_ + t.offset; }
    const std::vector<GgufTensor>& tensors() const { return tensors_; }
    uint64_t data_offset() const { return data_offset_; }
    uint64_t size() const { return len_; }

private:
    const uint8_t* base_ = nullptr;
    uint64_t len_ = 0;
    uint64_t data_offset_ = 0;
    std::map<std::string, GgufValue> kv_;
    std::vector<GgufTensor> tensors_;
    std::map<std::string, size_t> index_;
};

}  // namespace ribn

// GGUF v3 reader (see gguf.h for the reference semantics it follows).
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

#include "common.h"

namespace ribn {
namespace {

constexpr uint64_t kMaxString = 16ull * 1024 * 1024;
constexpr uint64_t kMaxArray = 1000000ull;
constexpr uint64_t kMaxTensors = 10000000ull;

struct Reader {
    const uint8_t* p;
    uint64_t len, pos = 0;
    std::string err;
    bool need(uint64_t n) {
        if (!err.empty()) return false;
        if (len - pos < n) { err = "GGUF file is truncated"; return false; }
        return true;
    }
    uint64_t uint(int n) {
        if (!need((uint64_t)n)) return 0;
        uint64_t v = 0;
        for (int i = 0; i < n; i++) v |= (uint64_t)p[pos + i] << (8 * i);
        pos += (uint64_t)n;
        return v;
    }
    std::string str() {
        uint64_t n = uint(8);
        if (!err.empty()) return {};
        if (n > kMaxString) { err = "GGUF string length " + std::to_string(n) + " exceeds the limit"; return {}; }
        if (!need(n)) return {};
        std::string s(reinterpret_cast<const char*>(p + pos), (size_t)n);
        pos += n;
        return s;
    }
};

void read_value(Reader& r, uint32_t type, GgufValue& v, int depth) {
    v.type = type;
    if (depth > 16) { r.err = "GGUF metadata arrays nest too deeply"; return; }
    switch (type) {
    case 0: v.u = r.uint(1); break;
    case 1: v.u = (uint64_t)(int64_t)(int8_t)r.uint(1); break;
    case 2: v.u = r.uint(2); break;
    case 3: v.u = (uint64_t)(int64_t)(int16_t)r.uint(2); break;
    case 4: v.u = r.uint(4); break;
    case 5: v.u = (uint64_t)(int64_t)(int32_t)r.uint(4); break;
    case 6: { uint32_t b = (uint32_t)r.uint(4); float f; std::memcpy(&f, &b, 4); v.f = f; break; }
    case 7: v.u = r.uint(1); if (r.err.empty() && v.u > 1) r.err = "invalid GGUF bool " + std::to_string(v.u); break;
    case 8: v.s = r.str(); break;
    case 9: {
        v.array_type = (uint32_t)r.uint(4);
        uint64_t n = r.uint(8);
        if (!r.err.empty()) return;
        if (n > kMaxArray) { r.err = "GGUF array length " + std::to_string(n) + " exceeds the limit"; return; }
        v.is_array = true;
        v.array_len = n;
        for (uint64_t i = 0; i < n && r.err.empty(); i++) {
            GgufValue tmp;
            read_value(r, v.array_type, tmp, depth + 1);
        }
        break;
    }
    case 10: case 11: v.u = r.uint(8); break;
    case 12: { uint64_t b = r.uint(8); double d; std::memcpy(&d, &b, 8); v.f = d; break; }
    default: r.err = "unsupported GGUF metadata type " + std::to_string(type); break;
    }
}

}  // namespace

GgufFile::~GgufFile() {
    if (base_) munmap(const_cast<uint8_t*>(base_), (size_t)len_);
}

std::string GgufFile::open(const std::string& path) {
    int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return "cannot open " + path + ": " + std::strerror(errno);
    struct stat st;
    if (fstat(fd, &st) != 0) { ::close(fd); return "cannot stat " + path; }
    len_ = (uint64_t)st.st_size;
    if (len_ == 0) { ::close(fd); return "GGUF file is truncated"; }
    void* m = mmap(nullptr, (size_t)len_, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) return "cannot map " + path;
    base_ = static_cast<const uint8_t*>(m);
    Reader r{base_, len_};
    uint32_t magic = (uint32_t)r.uint(4);
    if (!r.err.empty()) return r.err;
    if (magic != 0x46554747u) return "invalid GGUF magic " + std::to_string(magic);
    uint32_t version = (uint32_t)r.uint(4);
    if (!r.err.empty()) return r.err;
    if (version != 3) return "unsupported GGUF version " + std::to_string(version);
    uint64_t nt = r.uint(8);
    if (r.err.empty() && nt > kMaxTensors) return "GGUF tensor count " + std::to_string(nt) + " exceeds the limit";
    uint64_t nkv = r.uint(8);
    if (r.err.empty() && nkv > kMaxArray) return "GGUF metadata count " + std::to_string(nkv) + " exceeds the limit";
    for (uint64_t i = 0; i < nkv && r.err.empty(); i++) {
        std::string key = r.str();
        uint32_t type = (uint32_t)r.uint(4);
        if (!r.err.empty()) break;
        GgufValue v;
        read_value(r, type, v, 0);
        if (!r.err.empty()) break;
        if (!kv_.emplace(key, v).second) return "duplicate GGUF metadata key " + key;
    }
    if (!r.err.empty()) return r.err;
    for (uint64_t i = 0; i < nt && r.err.empty(); i++) {
        GgufTensor t;
        t.name = r.str();
        uint32_t nd = (uint32_t)r.uint(4);
        if (r.err.empty() && nd > 16) return "invalid tensor dimension count " + std::to_string(nd);
        for (uint32_t d = 0; d < nd; d++) t.dims.push_back(r.uint(8));
        t.type = (uint32_t)r.uint(4);
        t.offset = r.uint(8);
        if (!r.err.empty()) break;
        // a second tensor of one name would be unreachable by lookup: rejected
        if (index_.count(t.name)) return "duplicate tensor name " + t.name;
        index_[t.name] = tensors_.size();
        tensors_.push_back(std::move(t));
    }
    if (!r.err.empty()) return r.err;
    uint64_t alignment = 32;
    if (const GgufValue* a = get("general.alignment")) {
        if (a->is_array || a->type == 6 || a->type == 8 || a->type == 12) return "general.alignment has the wrong type";
        alignment = a->u;
    }
    if (alignment == 0 || (alignment & (alignment - 1))) return "invalid GGUF alignment " + std::to_string(alignment);
    uint64_t off = r.pos;
    if (off % alignment) off += alignment - off % alignment;
    if (off > len_) return "GGUF file is truncated";
    data_offset_ = off;
    for (auto& t : tensors_) {
        if (t.offset > len_ - off) return "tensor " + t.name + " offset " + std::to_string(t.offset) + " is out of bounds";
        uint64_t be, bb;
        if (type_layout(t.type, &be, &bb) && !t.dims.empty()) {
            // checked products, as TensorInfo::byte_len (crates/gguf/src/lib.rs:142-168):
            // an element count or byte length that overflows u64 is an error
            uint64_t n = 1;
            for (auto d : t.dims)
                if (__builtin_mul_overflow(n, d, &n)) return "tensor " + t.name + " element count overflows";
            if (t.dims[0] % be || n % be)
                return "tensor " + t.name + " dimension " + std::to_string(t.dims[0]) + " is not a multiple of " +
                       std::to_string(be);
            if (__builtin_mul_overflow(n / be, bb, &t.bytes)) return "tensor " + t.name + " byte length overflows";
            if (t.bytes > len_ - off - t.offset) return "tensor " + t.name + " extends past the end of the file";
        }
    }
    return {};
}

const GgufValue* GgufFile::get(const std::string& key) const {
    auto it = kv_.find(key);
    return it == kv_.end() ? nullptr : &it->second;
}
bool GgufFile::get_u64(const std::string& key, uint64_t* out) const {
    const GgufValue* v = get(key);
    if (!v || v->is_array || v->type == 6 || v->type == 8 || v->type == 12) return false;
    *out = v->u;
    return true;
}
bool GgufFile::get_f32(const std::string& key, float* out) const {
    const GgufValue* v = get(key);
    if (!v || (v->type != 6 && v->type != 12)) return false;
    *out = (float)v->f;
    return true;
}
bool GgufFile::get_str(const std::string& key, std::string* out) const {
    const GgufValue* v = get(key);
    if (!v || v->type != 8) return false;
    *out = v->s;
    return true;
}
const GgufTensor* GgufFile::tensor(const std::string& name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
}

}  // namespace ribn

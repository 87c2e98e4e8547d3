// Minimal JSON reader for model packages (config.json, the SafeTensors header):
// objects, arrays, strings (with \uXXXX escapes kept as UTF-8), numbers, booleans
// and null. Parse errors come back as a message naming the offset.
#pragma once
#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace ribn {
namespace json {

struct Value {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Value> arr;
    std::map<std::string, Value> obj;

    const Value* get(const std::string& k) const {
        if (kind != Object) return nullptr;
        auto it = obj.find(k);
        return it == obj.end() ? nullptr : &it->second;
    }
    bool is_number() const { return kind == Number; }
};

class Parser {
public:
    Parser(const char* p, size_t n) : p_(p), end_(p + n), begin_(p) {}
    bool parse(Value& out, std::string& err) {
        skip();
        if (!value(out, 0)) {
            err = "JSON parse error at offset " + std::to_string(p_ - begin_) + ": " + err_;
            return false;
        }
        skip();
        if (p_ != end_) {
            err = "JSON parse error: trailing data at offset " + std::to_string(p_ - begin_);
            return false;
        }
        return true;
    }

private:
    const char *p_, *end_, *begin_;
    std::string err_;
    void skip() {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) p_++;
    }
    bool fail(const char* m) {
        err_ = m;
        return false;
    }
    bool literal(const char* w) {
        const size_t n = std::char_traits<char>::length(w);
        if ((size_t)(end_ - p_) < n || std::string(p_, n) != w) return false;
        p_ += n;
        return true;
    }
    static void utf8(std::string& s, uint32_t cp) {
        if (cp < 0x80) s += (char)cp;
        else if (cp < 0x800) { s += (char)(0xC0 | (cp >> 6)); s += (char)(0x80 | (cp & 0x3F)); }
        else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12)); s += (char)(0x80 | ((cp >> 6) & 0x3F)); s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18)); s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F)); s += (char)(0x80 | (cp & 0x3F));
        }
    }
    bool hex4(uint32_t& v) {
        if (end_ - p_ < 4) return false;
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p_++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool string(std::string& s) {
        if (p_ >= end_ || *p_ != '"') return fail("expected a string");
        p_++;
        while (p_ < end_ && *p_ != '"') {
            char c = *p_++;
            if ((unsigned char)c < 0x20) return fail("control character in string");
            if (c != '\\') {
                s += c;
                continue;
            }
            if (p_ >= end_) return fail("unterminated escape");
            c = *p_++;
            switch (c) {
            case '"': s += '"'; break;
            case '\\': s += '\\'; break;
            case '/': s += '/'; break;
            case 'b': s += '\b'; break;
            case 'f': s += '\f'; break;
            case 'n': s += '\n'; break;
            case 'r': s += '\r'; break;
            case 't': s += '\t'; break;
            case 'u': {
                uint32_t cp;
                if (!hex4(cp)) return fail("bad \\u escape");
                if (cp >= 0xD800 && cp < 0xDC00 && end_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
                    p_ += 2;
                    uint32_t lo;
                    if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                utf8(s, cp);
                break;
            }
            default: return fail("unknown escape");
            }
        }
        if (p_ >= end_) return fail("unterminated string");
        p_++;
        return true;
    }
    bool value(Value& v, int depth) {
        if (depth > 64) return fail("nesting too deep");
        skip();
        if (p_ >= end_) return fail("unexpected end");
        const char c = *p_;
        if (c == '{') {
            p_++;
            v.kind = Value::Object;
            skip();
            if (p_ < end_ && *p_ == '}') { p_++; return true; }
            for (;;) {
                skip();
                std::string key;
                if (!string(key)) return false;
                skip();
                if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
                p_++;
                Value item;
                if (!value(item, depth + 1)) return false;
                v.obj[key] = std::move(item);
                skip();
                if (p_ < end_ && *p_ == ',') { p_++; continue; }
                if (p_ < end_ && *p_ == '}') { p_++; return true; }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            p_++;
            v.kind = Value::Array;
            skip();
            if (p_ < end_ && *p_ == ']') { p_++; return true; }
            for (;;) {
                Value item;
                if (!value(item, depth + 1)) return false;
                v.arr.push_back(std::move(item));
                skip();
                if (p_ < end_ && *p_ == ',') { p_++; continue; }
                if (p_ < end_ && *p_ == ']') { p_++; return true; }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') {
            v.kind = Value::String;
            return string(v.str);
        }
        if (literal("true")) { v.kind = Value::Bool; v.b = true; return true; }
        if (literal("false")) { v.kind = Value::Bool; v.b = false; return true; }
        if (literal("null")) { v.kind = Value::Null; return true; }
        if (c == '-' || (c >= '0' && c <= '9')) {
            const char* s = p_;
            if (*p_ == '-') p_++;
            while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                                 *p_ == '+' || *p_ == '-'))
                p_++;
            const std::string t(s, p_);
            char* e = nullptr;
            v.kind = Value::Number;
            v.num = std::strtod(t.c_str(), &e);
            if (!e || *e) return fail("bad number");
            return true;
        }
        return fail("unexpected character");
    }
};

inline bool parse(const std::string& text, Value& out, std::string& err) {
    Parser p(text.data(), text.size());
    return p.parse(out, err);
}

}  // namespace json
}  // namespace ribn

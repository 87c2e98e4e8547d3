// Shared host-side helpers for librocm_ribn (no device code here).
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <string>

namespace ribn {

// GGML value types used on the token loop (crates/gguf/src/lib.rs:508-535).
enum GgmlType : uint32_t {
    GGML_F32 = 0,
    GGML_F16 = 1,
    GGML_Q8_0 = 8,
    GGML_Q4_K = 12,
    GGML_Q6_K = 14,
};

// (block elements, block bytes); false for a type without a layout here.
inline bool type_layout(uint32_t t, uint64_t* be, uint64_t* bb) {
    switch (t) {
    case GGML_F32: *be = 1; *bb = 4; return true;
    case GGML_F16: *be = 1; *bb = 2; return true;
    case GGML_Q8_0: *be = 32; *bb = 34; return true;
    case GGML_Q4_K: *be = 256; *bb = 144; return true;
    case GGML_Q6_K: *be = 256; *bb = 210; return true;
    default: return false;
    }
}

inline const char* type_name(uint32_t t) {
    switch (t) {
    case GGML_F32: return "F32";
    case GGML_F16: return "F16";
    case GGML_Q8_0: return "Q8_0";
    case GGML_Q4_K: return "Q4_K";
    case GGML_Q6_K: return "Q6_K";
    default: return "unsupported";
    }
}

// binary32 -> binary16, round to nearest even (overflow -> inf, NaN kept quiet).
inline uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds to >= 65520
    if (ax < 0x38800000u) {                                     // f16 subnormal or zero
        if (ax < 0x33000000u) return (uint16_t)sign;            // < 2^-25 -> 0
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        int e = (int)(ax >> 23);                                // 102..112
        int shift = 126 - e;                                    // 14..24
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

inline float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, x;
    if (e == 0) {
        if (m == 0) x = sign;
        else {
            int s = 0;
            while (!(m & 0x400u)) { m <<= 1; s++; }
            m &= 0x3ffu;
            x = sign | ((uint32_t)(113 - s) << 23) | (m << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

// Bounded diagnostic copy: at most err_len-1 bytes plus NUL (executor.rs:134-152
// bounds retained diagnostics to 4096 bytes).
inline void set_err(char* err, size_t err_len, const std::string& msg) {
    if (!err || err_len == 0) return;
    size_t n = msg.size();
    if (n > err_len - 1) n = err_len - 1;
    if (n > 4095) n = 4095;
    std::memcpy(err, msg.data(), n);
    err[n] = 0;
}

}  // namespace ribn

// test_common.h -- helpers shared by the C++ test programs (fp16 bit
// conversions as the reference's tests spell them, tests/test_matmul_w4a16.cpp:23-54).
#pragma once

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace t {

// Truncating encode, as the reference tests build their fp16 inputs.
inline uint16_t f2h(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t e = static_cast<int32_t>((x >> 23) & 0xff) - 127 + 15;
    const uint32_t m = x & 0x7fffffu;
    if (e <= 0) return static_cast<uint16_t>(sign);
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e) << 10) | (m >> 13));
}

inline float h2f(uint16_t h) {
    const uint32_t sign = (static_cast<uint32_t>(h) & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t out;
    if (e == 0) {
        if (m == 0) out = sign;
        else {
            const float v = static_cast<float>(m) * 5.9604644775390625e-08f;
            return sign ? -v : v;
        }
    } else if (e == 31) {
        out = sign | 0x7f800000u | (m << 13);
    } else {
        out = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &out, 4);
    return f;
}

// IEEE round-to-nearest-even encode with subnormals (the kernels' rounding).
inline uint16_t f2h_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return static_cast<uint16_t>(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    const int32_t e = static_cast<int32_t>(ax >> 23) - 127;
    if (e > 15) return static_cast<uint16_t>(sign | 0x7c00u);
    if (e >= -14) {
        const uint32_t frac = ax & 0x7fffffu, q = frac >> 13, rem = frac & 0x1fffu;
        uint32_t r = (static_cast<uint32_t>(e + 15) << 10) + q;
        if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++r;
        return static_cast<uint16_t>(sign | r);
    }
    if (ax == 0) return static_cast<uint16_t>(sign);
    const int32_t shift = -e - 1;
    if (shift > 25) return static_cast<uint16_t>(sign);
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return static_cast<uint16_t>(sign | q);
}

inline int fail(const char* fmt, const char* what) {
    std::fprintf(stderr, fmt, what);
    return 1;
}

// Writes a safetensors file from (name, dtype, shape, bytes) entries.
struct StEntry {
    std::string name, dtype;
    std::vector<int64_t> shape;
    std::vector<uint8_t> bytes;
};

inline void write_safetensors(const std::string& path, const std::vector<StEntry>& entries, bool with_metadata = true) {
    std::string h = "{";
    if (with_metadata) h += "\"__metadata__\":{\"format\":\"pt\",\"nested\":{\"a\":[1,2]}},";
    uint64_t off = 0;
    for (size_t i = 0; i < entries.size(); ++i) {
        const auto& e = entries[i];
        h += "\"" + e.name + "\":{\"dtype\":\"" + e.dtype + "\",\"shape\":[";
        for (size_t j = 0; j < e.shape.size(); ++j) h += (j ? "," : "") + std::to_string(e.shape[j]);
        h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + e.bytes.size()) + "]}";
        off += e.bytes.size();
        if (i + 1 < entries.size()) h += ",";
    }
    h += "}";
    FILE* f = std::fopen(path.c_str(), "wb");
    const uint64_t n = h.size();
    std::fwrite(&n, 8, 1, f);
    std::fwrite(h.data(), 1, h.size(), f);
    for (const auto& e : entries) std::fwrite(e.bytes.data(), 1, e.bytes.size(), f);
    std::fclose(f);
}

template <typename T>
std::vector<uint8_t> bytes_of(const std::vector<T>& v) {
    std::vector<uint8_t> b(v.size() * sizeof(T));
    std::memcpy(b.data(), v.data(), b.size());
    return b;
}

}  // namespace t

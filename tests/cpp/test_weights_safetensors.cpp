// CPU-only: the safetensors index parses what the format allows (metadata,
// every supported dtype including I8, zero-sized tensors), exposes host bytes,
// and rejects malformed files with an exception (the reference's loader
// throws the same way, src/csrc/lib/weights.cpp:264-334).
#include "minicpmv/weights.h"
#include "test_common.h"

#include <stdexcept>

using namespace minicpmv;

static bool throws(const std::string& path) {
    try {
        WeightsIndex idx(path);
    } catch (const std::runtime_error& e) {
        std::printf("  rejected %s: %s\n", path.c_str(), e.what());
        return true;
    }
    return false;
}

static void raw(const std::string& path, const std::string& header, size_t data_bytes, bool lie_len = false) {
    FILE* f = std::fopen(path.c_str(), "wb");
    uint64_t n = lie_len ? header.size() + 100 : header.size();
    std::fwrite(&n, 8, 1, f);
    std::fwrite(header.data(), 1, header.size(), f);
    std::vector<uint8_t> z(data_bytes, 0);
    if (data_bytes) std::fwrite(z.data(), 1, z.size(), f);
    std::fclose(f);
}

int main(int argc, char** argv) {
    const std::string dir = argc > 1 ? argv[1] : "/tmp";
    const std::string p = dir + "/mcv_test.safetensors";
    std::vector<int32_t> i32 = {1, -2, 3, 0x76543210};
    std::vector<int8_t> i8 = {-128, -1, 0, 127, 5, 6};
    std::vector<uint16_t> f16 = {0x3c00, 0xbc00};
    std::vector<uint16_t> bf16 = {0x3f80, 0x4000, 0x0001};    // 1.0, 2.0, tiny
    t::write_safetensors(p, {{"a.qweight", "I32", {2, 2}, t::bytes_of(i32)},
                             {"a.i8", "I8", {2, 3}, t::bytes_of(i8)},
                             {"a.scales", "F16", {1, 2}, t::bytes_of(f16)},
                             {"b.bf16", "BF16", {3}, t::bytes_of(bf16)},
                             {"empty", "F32", {0, 4}, {}}});
    WeightsIndex idx(p);
    int rc = 0;
    if (idx.size() != 5 || !idx.contains("a.i8") || idx.contains("__metadata__")) rc = 1;
    const TensorInfo& qi = idx.at("a.qweight");
    if (qi.dtype != DType::Int32 || qi.shape != std::vector<int64_t>{2, 2}) rc = 1;
    if (idx.at("a.i8").dtype != DType::Int8) rc = 1;
    int32_t w3;
    std::memcpy(&w3, idx.host_data("a.qweight") + 12, 4);
    if (w3 != 0x76543210) rc = 1;
    if (reinterpret_cast<const int8_t*>(idx.host_data("a.i8"))[0] != -128) rc = 1;
    if (idx.names().front() != "a.i8") rc = 1;
    if (idx.at("empty").data_end != idx.at("empty").data_begin) rc = 1;
    try {
        (void)idx.at("missing");
        rc = 1;
    } catch (const std::runtime_error&) {
    }
    std::printf("valid file parsed: rc=%d\n", rc);

    raw(dir + "/bad1.safetensors", "{\"x\":{\"dtype\":\"F16\",\"shape\":[2],\"data_offsets\":[0,4]}", 4);   // no closing brace
    raw(dir + "/bad2.safetensors", "{\"x\":{\"dtype\":\"Q4\",\"shape\":[2],\"data_offsets\":[0,4]}}", 4);  // unknown dtype
    raw(dir + "/bad3.safetensors", "{\"x\":{\"dtype\":\"F16\",\"shape\":[3],\"data_offsets\":[0,4]}}", 4); // size mismatch
    raw(dir + "/bad4.safetensors", "{\"x\":{\"dtype\":\"F16\",\"shape\":[2],\"data_offsets\":[0,40]}}", 4); // past EOF
    raw(dir + "/bad5.safetensors", "{\"x\":{\"dtype\":\"F16\",\"shape\":[2]}}", 4);                       // no offsets
    raw(dir + "/bad6.safetensors", "{}", 0, true);                                                           // header length lies
    // data_offsets whose sum with the data section's start wraps past 2^64
    // (into the header, with a size that matches the shape)
    raw(dir + "/bad8.safetensors", "{\"x\":{\"dtype\":\"F16\",\"shape\":[2],\"data_offsets\":[18446744073709551608,18446744073709551612]}}", 4);
    // a shape whose element count wraps to 0 with empty data
    raw(dir + "/bad9.safetensors", "{\"x\":{\"dtype\":\"F16\",\"shape\":[4294967296,4294967296],\"data_offsets\":[0,0]}}", 0);
    // a shape dimension above INT64_MAX
    raw(dir + "/bad10.safetensors", "{\"x\":{\"dtype\":\"U8\",\"shape\":[9223372036854775808,2],\"data_offsets\":[0,0]}}", 0);
    // metadata nested a million levels deep (refused, not recursed into)
    raw(dir + "/bad11.safetensors", "{\"__metadata__\":" + std::string(1000000, '[') + std::string(1000000, ']') + "}", 0);
    for (int i : {1, 2, 3, 4, 5, 6, 8, 9, 10, 11})
        if (!throws(dir + "/bad" + std::to_string(i) + ".safetensors")) {
            std::printf("bad%d accepted\n", i);
            rc = 1;
        }
    FILE* f = std::fopen((dir + "/bad7.safetensors").c_str(), "wb");
    std::fwrite("abc", 1, 3, f);
    std::fclose(f);
    if (!throws(dir + "/bad7.safetensors")) rc = 1;
    if (!throws(dir + "/does_not_exist.safetensors")) rc = 1;
    std::printf("%s\n", rc ? "FAILED" : "ok");
    return rc;
}

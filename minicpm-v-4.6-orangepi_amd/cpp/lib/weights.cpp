// weights.cpp -- memory-mapped safetensors index.
//
// File format: 8-byte little-endian header length, a JSON object mapping
// tensor names to {"dtype", "shape", "data_offsets": [begin, end]} (plus an
// optional "__metadata__" object), then the raw data.  The parser below reads
// only what that format needs and rejects anything malformed with a message.
#include "minicpmv/weights.h"

#include "minicpmv/hip_context.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cctype>
#include <cstdlib>
#include <cstring>
#include <stdexcept>

namespace minicpmv {
namespace {

DType dtype_from_string(const std::string& s) {
    if (s == "F16") return DType::Float16;
    if (s == "BF16") return DType::BFloat16;
    if (s == "F32") return DType::Float32;
    if (s == "I32") return DType::Int32;
    if (s == "I64") return DType::Int64;
    if (s == "U8") return DType::UInt8;
    if (s == "I8") return DType::Int8;
    throw std::runtime_error("unsupported safetensors dtype: " + s);
}

// Truncating bf16 -> fp16, as the reference loads bf16 weights
// (src/csrc/lib/weights.cpp:25-33).
uint16_t bf16_to_f16_trunc(uint16_t bf) {
    const uint32_t bits = static_cast<uint32_t>(bf) << 16;
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int32_t e = static_cast<int32_t>((bits >> 23) & 0xffu) - 112;
    if (e <= 0) return static_cast<uint16_t>(sign);
    if (e >= 31) return static_cast<uint16_t>(sign | 0x7c00u);
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(e) << 10) | ((bits & 0x7fffffu) >> 13));
}

class HeaderParser {
public:
    explicit HeaderParser(const std::string& s) : s_(s) {}

    void ws() {
        while (i_ < s_.size() && std::isspace(static_cast<unsigned char>(s_[i_]))) ++i_;
    }
    bool peek(char c) {
        ws();
        return i_ < s_.size() && s_[i_] == c;
    }
    void expect(char c) {
        ws();
        if (i_ >= s_.size() || s_[i_] != c)
            throw std::runtime_error(std::string("safetensors header: expected '") + c + "' at offset " + std::to_string(i_));
        ++i_;
    }
    std::string str() {
        expect('"');
        std::string out;
        while (i_ < s_.size() && s_[i_] != '"') {
            if (s_[i_] == '\\') {
                if (i_ + 1 >= s_.size()) break;
                out.push_back(s_[i_ + 1]);
                i_ += 2;
            } else {
                out.push_back(s_[i_++]);
            }
        }
        expect('"');
        return out;
    }
    uint64_t uint() {
        ws();
        if (i_ >= s_.size() || !std::isdigit(static_cast<unsigned char>(s_[i_])))
            throw std::runtime_error("safetensors header: expected an unsigned integer at offset " + std::to_string(i_));
        uint64_t v = 0;
        while (i_ < s_.size() && std::isdigit(static_cast<unsigned char>(s_[i_]))) {
            const uint64_t d = static_cast<uint64_t>(s_[i_++] - '0');
            if (v > (UINT64_MAX - d) / 10) throw std::runtime_error("safetensors header: integer overflow");
            v = v * 10 + d;
        }
        return v;
    }
    std::vector<uint64_t> uint_array() {
        std::vector<uint64_t> out;
        expect('[');
        if (peek(']')) { ++i_; return out; }
        for (;;) {
            out.push_back(uint());
            if (peek(',')) { ++i_; continue; }
            expect(']');
            return out;
        }
    }
    // Skips any JSON value (used for __metadata__ and unknown keys); nesting
    // deeper than kMaxDepth is refused rather than recursed into.
    void skip_value(int depth = 0) {
        ws();
        if (i_ >= s_.size()) throw std::runtime_error("safetensors header: truncated");
        const char c = s_[i_];
        if (c == '"') { (void)str(); return; }
        if (c == '{' || c == '[') {
            if (depth >= kMaxDepth)
                throw std::runtime_error("safetensors header: values nested deeper than " + std::to_string(kMaxDepth));
            const char close = c == '{' ? '}' : ']';
            ++i_;
            if (peek(close)) { ++i_; return; }
            for (;;) {
                if (c == '{') { (void)str(); expect(':'); }
                skip_value(depth + 1);
                if (peek(',')) { ++i_; continue; }
                expect(close);
                return;
            }
        }
        while (i_ < s_.size() && s_[i_] != ',' && s_[i_] != '}' && s_[i_] != ']') ++i_;
    }
    bool at_end() {
        ws();
        return i_ >= s_.size();
    }

private:
    static constexpr int kMaxDepth = 64;
    const std::string& s_;
    size_t i_{0};
};

}  // namespace

WeightsIndex::WeightsIndex(const std::string& safetensors_path) : path_(safetensors_path) {
    const int fd = ::open(path_.c_str(), O_RDONLY);
    if (fd < 0) throw std::runtime_error("failed to open safetensors file: " + path_);
    struct stat st;
    if (::fstat(fd, &st) != 0) {
        ::close(fd);
        throw std::runtime_error("failed to stat safetensors file: " + path_);
    }
    map_size_ = static_cast<size_t>(st.st_size);
    if (map_size_ > 0) {
        void* p = ::mmap(nullptr, map_size_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            ::close(fd);
            throw std::runtime_error("failed to map safetensors file: " + path_);
        }
        map_ = static_cast<const uint8_t*>(p);
    }
    ::close(fd);
    try {
        parse();
    } catch (...) {
        if (map_) ::munmap(const_cast<uint8_t*>(map_), map_size_);
        map_ = nullptr;
        throw;
    }
}

WeightsIndex::~WeightsIndex() {
    if (map_) ::munmap(const_cast<uint8_t*>(map_), map_size_);
}

void WeightsIndex::parse() {
    if (map_size_ < 8) throw std::runtime_error("invalid safetensors file (shorter than 8 bytes): " + path_);
    uint64_t header_len = 0;
    std::memcpy(&header_len, map_, 8);
    if (header_len > map_size_ - 8) throw std::runtime_error("invalid safetensors header length: " + path_);
    const std::string header(reinterpret_cast<const char*>(map_ + 8), static_cast<size_t>(header_len));
    const uint64_t data_base = 8 + header_len;
    HeaderParser p(header);
    p.expect('{');
    if (p.peek('}')) { p.expect('}'); return; }
    for (;;) {
        const std::string name = p.str();
        p.expect(':');
        if (name == "__metadata__") {
            p.skip_value();
        } else {
            TensorInfo info{};
            bool have_dtype = false, have_shape = false, have_offsets = false;
            p.expect('{');
            for (;;) {
                const std::string key = p.str();
                p.expect(':');
                if (key == "dtype") {
                    info.dtype = dtype_from_string(p.str());
                    have_dtype = true;
                } else if (key == "shape") {
                    for (uint64_t d : p.uint_array()) {
                        if (d > static_cast<uint64_t>(INT64_MAX)) throw std::runtime_error("bad shape for " + name);
                        info.shape.push_back(static_cast<int64_t>(d));
                    }
                    have_shape = true;
                } else if (key == "data_offsets") {
                    const auto off = p.uint_array();
                    // offsets are relative to the data section and end inside the file
                    if (off.size() != 2 || off[0] > off[1] || off[1] > map_size_ - data_base)
                        throw std::runtime_error("bad data_offsets for " + name);
                    info.data_begin = data_base + off[0];
                    info.data_end = data_base + off[1];
                    have_offsets = true;
                } else {
                    p.skip_value();
                }
                if (p.peek(',')) { p.expect(','); continue; }
                p.expect('}');
                break;
            }
            if (!have_dtype || !have_shape || !have_offsets)
                throw std::runtime_error("incomplete tensor entry for " + name);
            if (info.data_end > map_size_) throw std::runtime_error("tensor data beyond end of file for " + name);
            uint64_t numel = 1;
            for (int64_t d : info.shape) {
                const uint64_t u = static_cast<uint64_t>(d);
                if (u != 0 && numel > UINT64_MAX / u / 8) throw std::runtime_error("shape too large for " + name);
                numel *= u;
            }
            if (numel * dtype_size(info.dtype) != info.data_end - info.data_begin)
                throw std::runtime_error("tensor byte size does not match its shape for " + name);
            tensors_.emplace(name, std::move(info));
        }
        if (p.peek(',')) { p.expect(','); continue; }
        p.expect('}');
        break;
    }
    if (!p.at_end()) throw std::runtime_error("trailing bytes after safetensors header");
}

const TensorInfo& WeightsIndex::at(const std::string& name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) throw std::runtime_error("tensor not found in " + path_ + ": " + name);
    return it->second;
}

bool WeightsIndex::contains(const std::string& name) const { return tensors_.count(name) != 0; }

std::vector<std::string> WeightsIndex::names() const {
    std::vector<std::string> out;
    out.reserve(tensors_.size());
    for (const auto& kv : tensors_) out.push_back(kv.first);
    std::sort(out.begin(), out.end());
    return out;
}

const uint8_t* WeightsIndex::host_data(const std::string& name) const { return map_ + at(name).data_begin; }

Tensor WeightsIndex::load_to_device(const std::string& name) const {
    const TensorInfo& info = at(name);
    Tensor t(info.shape, info.dtype);
    t.allocate();
    if (info.data_end > info.data_begin) t.copy_from_host(map_ + info.data_begin, info.data_end - info.data_begin);
    return t;
}

Tensor WeightsIndex::load_to_device_as(const std::string& name, DType target) const {
    const TensorInfo& info = at(name);
    if (info.dtype == target) return load_to_device(name);
    if (!(info.dtype == DType::BFloat16 && target == DType::Float16))
        throw std::runtime_error("unsupported dtype conversion in load_to_device_as");
    const size_t n = (info.data_end - info.data_begin) / 2;
    std::vector<uint16_t> conv(n);
    const uint8_t* src = map_ + info.data_begin;
    for (size_t i = 0; i < n; ++i) {
        uint16_t v;
        std::memcpy(&v, src + 2 * i, 2);
        conv[i] = bf16_to_f16_trunc(v);
    }
    Tensor t(info.shape, target);
    t.copy_from_host(conv.data(), conv.size() * 2);
    return t;
}

std::string default_safetensors_path() {
    if (const char* env = std::getenv("MINICPMV_MODEL_PATH")) {
        if (*env) return std::string(env) + "/model.safetensors";
    }
    return "./MiniCPM-V-4.6/model.safetensors";
}

}  // namespace minicpmv

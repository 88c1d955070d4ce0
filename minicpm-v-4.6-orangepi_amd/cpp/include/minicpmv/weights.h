// weights.h -- safetensors index.
//
// Mirrors WeightsIndex (src/csrc/include/minicpmv/weights.h:19-42) with two
// differences: the file is memory-mapped instead of read whole, and I8 is a
// supported dtype (the reference's parse_dtype has no I8,
// src/csrc/lib/weights.cpp:15-23).  host_data() exposes tensor bytes on the
// host so packers need no device round trip (quantized_weight.cpp:27-39).
#pragma once

#include "minicpmv/tensor.h"

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace minicpmv {

struct TensorInfo {
    DType dtype;
    std::vector<int64_t> shape;
    uint64_t data_begin;
    uint64_t data_end;
};

class WeightsIndex {
public:
    explicit WeightsIndex(const std::string& safetensors_path);
    ~WeightsIndex();
    WeightsIndex(const WeightsIndex&) = delete;
    WeightsIndex& operator=(const WeightsIndex&) = delete;

    const TensorInfo& at(const std::string& name) const;
    bool contains(const std::string& name) const;
    size_t size() const { return tensors_.size(); }
    std::vector<std::string> names() const;

    // Host view of a tensor's bytes inside the mapped file.
    const uint8_t* host_data(const std::string& name) const;

    Tensor load_to_device(const std::string& name) const;
    // BF16 -> F16 uses the reference's truncating conversion (weights.cpp:25-33).
    Tensor load_to_device_as(const std::string& name, DType target_dtype) const;

private:
    std::string path_;
    const uint8_t* map_{nullptr};
    size_t map_size_{0};
    std::unordered_map<std::string, TensorInfo> tensors_;

    void parse();
};

// MINICPMV_MODEL_PATH/model.safetensors, else ./MiniCPM-V-4.6/model.safetensors
// (src/csrc/lib/weights.cpp:336-343).
std::string default_safetensors_path();

}  // namespace minicpmv

// tensor.cpp -- hipMalloc-backed device buffers and tensors.
#include "minicpmv/tensor.h"

#include "minicpmv/hip_context.h"

#include <hip/hip_runtime_api.h>

#include <numeric>
#include <stdexcept>

namespace minicpmv {

size_t dtype_size(DType dtype) {
    switch (dtype) {
        case DType::Float16:
        case DType::BFloat16: return 2;
        case DType::Float32:
        case DType::Int32: return 4;
        case DType::Int64: return 8;
        case DType::UInt8:
        case DType::Int8: return 1;
    }
    throw std::runtime_error("unknown dtype");
}

const char* dtype_name(DType dtype) {
    switch (dtype) {
        case DType::Float16: return "F16";
        case DType::BFloat16: return "BF16";
        case DType::Float32: return "F32";
        case DType::Int32: return "I32";
        case DType::Int64: return "I64";
        case DType::UInt8: return "U8";
        case DType::Int8: return "I8";
    }
    return "?";
}

DeviceBuffer::DeviceBuffer(size_t bytes) { allocate(bytes); }

DeviceBuffer::~DeviceBuffer() { reset(); }

DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept : data_(other.data_), size_bytes_(other.size_bytes_) {
    other.data_ = nullptr;
    other.size_bytes_ = 0;
}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept {
    if (this != &other) {
        reset();
        data_ = other.data_;
        size_bytes_ = other.size_bytes_;
        other.data_ = nullptr;
        other.size_bytes_ = 0;
    }
    return *this;
}

void DeviceBuffer::allocate(size_t bytes) {
    reset();
    if (bytes == 0) return;
    check_hip(hipMalloc(&data_, bytes), "hipMalloc");
    size_bytes_ = bytes;
}

void DeviceBuffer::reset() {
    if (data_ != nullptr) {
        (void)hipFree(data_);
        data_ = nullptr;
        size_bytes_ = 0;
    }
}

Tensor::Tensor(std::vector<int64_t> shape, DType dtype) : shape_(std::move(shape)), dtype_(dtype) {
    for (int64_t d : shape_)
        if (d < 0) throw std::runtime_error("Tensor: negative dimension");
}

void Tensor::allocate() { buffer_.allocate(size_bytes()); }

void Tensor::copy_from_host(const void* src, size_t bytes) {
    if (bytes > size_bytes()) throw std::runtime_error("Tensor::copy_from_host: more bytes than the tensor holds");
    if (buffer_.data() == nullptr) allocate();
    check_hip(hipMemcpy(buffer_.data(), src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

void Tensor::copy_to_host(void* dst, size_t bytes) const {
    if (bytes > buffer_.size_bytes()) throw std::runtime_error("Tensor::copy_to_host: more bytes than allocated");
    check_hip(hipMemcpy(dst, buffer_.data(), bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

void Tensor::zero() {
    if (buffer_.data() == nullptr) allocate();
    if (size_bytes() != 0) check_hip(hipMemset(buffer_.data(), 0, size_bytes()), "hipMemset");
}

size_t Tensor::numel() const {
    if (shape_.empty()) return 0;
    return std::accumulate(shape_.begin(), shape_.end(), size_t{1},
                           [](size_t a, int64_t b) { return a * static_cast<size_t>(b); });
}

size_t Tensor::size_bytes() const { return numel() * dtype_size(dtype_); }

}  // namespace minicpmv

// tensor.cpp -- device memory ownership for the operator surface.
//
// DeviceBuffer owns one hipMalloc allocation through a unique_ptr whose
// deleter calls hipFree, so moves, resets and destruction are the smart
// pointer's; Tensor adds a validated shape and dtype and allocates lazily.
// Element counts are checked for overflow when a shape is set, so every later
// size computation is exact.
#include "minicpmv/tensor.h"

#include "minicpmv/hip_context.h"

#include <hip/hip_runtime_api.h>

#include <limits>
#include <stdexcept>
#include <string>
#include <utility>

namespace minicpmv {
namespace {

struct DTypeInfo {
    size_t bytes;
    const char* name;
};

// Indexed by the DType enumerators in declaration order.
constexpr DTypeInfo kDTypes[] = {
    {2, "F16"},  // Float16
    {2, "BF16"}, // BFloat16
    {4, "F32"},  // Float32
    {4, "I32"},  // Int32
    {8, "I64"},  // Int64
    {1, "U8"},   // UInt8
    {1, "I8"},   // Int8
};

const DTypeInfo& info(DType dtype) {
    const auto i = static_cast<size_t>(dtype);
    if (i >= sizeof(kDTypes) / sizeof(kDTypes[0])) throw std::runtime_error("unknown dtype");
    return kDTypes[i];
}

// Product of the dimensions; 0 for an empty shape (the reference's convention
// for a default-constructed tensor); throws on a negative dimension or a
// product that does not fit in size_t.
size_t checked_numel(const std::vector<int64_t>& shape) {
    if (shape.empty()) return 0;
    size_t n = 1;
    for (int64_t d : shape) {
        if (d < 0) throw std::runtime_error("Tensor: negative dimension " + std::to_string(d));
        const auto u = static_cast<size_t>(d);
        if (u != 0 && n > std::numeric_limits<size_t>::max() / u)
            throw std::runtime_error("Tensor: element count overflows");
        n *= u;
    }
    return n;
}

}  // namespace

size_t dtype_size(DType dtype) { return info(dtype).bytes; }

const char* dtype_name(DType dtype) { return info(dtype).name; }

void DeviceBuffer::HipFree::operator()(void* p) const noexcept { (void)hipFree(p); }

DeviceBuffer::DeviceBuffer(size_t bytes) { allocate(bytes); }

DeviceBuffer::DeviceBuffer(DeviceBuffer&& other) noexcept
    : mem_(std::move(other.mem_)), size_bytes_(std::exchange(other.size_bytes_, 0)) {}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& other) noexcept {
    if (this != &other) {
        mem_ = std::move(other.mem_);               // frees what this buffer held
        size_bytes_ = std::exchange(other.size_bytes_, 0);
    }
    return *this;
}

void DeviceBuffer::allocate(size_t bytes) {
    reset();
    if (bytes == 0) return;
    void* p = nullptr;
    check_hip(hipMalloc(&p, bytes), "hipMalloc");
    mem_.reset(p);
    size_bytes_ = bytes;
}

void DeviceBuffer::reset() {
    mem_.reset();
    size_bytes_ = 0;
}

Tensor::Tensor(std::vector<int64_t> shape, DType dtype)
    : shape_(std::move(shape)), dtype_(dtype), numel_(checked_numel(shape_)) {
    if (numel_ > std::numeric_limits<size_t>::max() / dtype_size(dtype_))
        throw std::runtime_error("Tensor: byte size overflows");
}

Tensor Tensor::view(const Tensor& storage, std::vector<int64_t> shape, DType dtype) {
    Tensor t(std::move(shape), dtype);
    if (storage.data() == nullptr) throw std::runtime_error("Tensor::view: storage is not allocated");
    if (t.size_bytes() > storage.size_bytes())
        throw std::runtime_error("Tensor::view: " + std::to_string(t.size_bytes()) + " bytes over a tensor of " +
                                 std::to_string(storage.size_bytes()));
    t.borrowed_ = storage.data();
    return t;
}

void Tensor::allocate() {
    if (borrowed_ != nullptr) throw std::runtime_error("Tensor::allocate: a view owns no memory");
    buffer_.allocate(size_bytes());
}

void Tensor::copy_from_host(const void* src, size_t bytes) {
    if (bytes > size_bytes())
        throw std::runtime_error("Tensor::copy_from_host: " + std::to_string(bytes) + " bytes into a tensor of " +
                                 std::to_string(size_bytes()));
    if (data() == nullptr) allocate();
    if (bytes != 0) check_hip(hipMemcpy(data(), src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

void Tensor::copy_to_host(void* dst, size_t bytes) const {
    const size_t have = borrowed_ != nullptr ? size_bytes() : buffer_.size_bytes();
    if (bytes > have)
        throw std::runtime_error("Tensor::copy_to_host: " + std::to_string(bytes) + " bytes from an allocation of " +
                                 std::to_string(have));
    if (bytes != 0) check_hip(hipMemcpy(dst, data(), bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

void Tensor::zero() {
    if (data() == nullptr) allocate();
    if (size_bytes() != 0) check_hip(hipMemset(data(), 0, size_bytes()), "hipMemset");
}

size_t Tensor::numel() const { return numel_; }

size_t Tensor::size_bytes() const { return numel_ * dtype_size(dtype_); }

}  // namespace minicpmv

// tensor.h -- device tensors over hipMalloc.
//
// Keeps the public surface of the reference's substrate
// (src/csrc/include/minicpmv/tensor.h:12-66): the same DType set, a move-only
// DeviceBuffer, and a Tensor that allocates lazily on its first
// copy_from_host.  The implementation is this build's own: the buffer is a
// unique_ptr with a hipFree deleter, and shapes are validated (no negative
// dimension, no overflowing element count) when a tensor is constructed.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

namespace minicpmv {

enum class DType {
    Float16,
    BFloat16,
    Float32,
    Int32,
    Int64,
    UInt8,
    Int8,
};

size_t dtype_size(DType dtype);
const char* dtype_name(DType dtype);

class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes);

    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    // A moved-from buffer is empty (no allocation, size 0).
    DeviceBuffer(DeviceBuffer&& other) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept;

    // Replaces any current allocation with `bytes` of device memory (none for 0).
    void allocate(size_t bytes);
    void reset();

    void* data() const { return mem_.get(); }
    size_t size_bytes() const { return size_bytes_; }

private:
    struct HipFree {
        void operator()(void* p) const noexcept;
    };
    std::unique_ptr<void, HipFree> mem_;
    size_t size_bytes_{0};
};

class Tensor {
public:
    Tensor() = default;
    Tensor(std::vector<int64_t> shape, DType dtype);

    // A non-owning tensor of `shape` and `dtype` over the start of `storage`'s
    // allocation (which must hold at least its bytes and must outlive it):
    // scratch memory reused under the shapes the operators validate.
    static Tensor view(const Tensor& storage, std::vector<int64_t> shape, DType dtype);

    void allocate();
    // Synchronous copies (legacy default stream, which orders after work
    // queued on blocking streams); the first copy_from_host allocates.
    void copy_from_host(const void* src, size_t bytes);
    void copy_to_host(void* dst, size_t bytes) const;
    // Fills the allocation with zero bytes (allocating it if needed).
    void zero();

    const std::vector<int64_t>& shape() const { return shape_; }
    DType dtype() const { return dtype_; }
    size_t numel() const;
    size_t size_bytes() const;
    void* data() const { return borrowed_ != nullptr ? borrowed_ : buffer_.data(); }
    bool is_view() const { return borrowed_ != nullptr; }

private:
    std::vector<int64_t> shape_;
    DType dtype_{DType::Float16};
    size_t numel_{0};
    DeviceBuffer buffer_;
    void* borrowed_{nullptr};      // set for views: memory owned by another tensor
};

}  // namespace minicpmv

// hip_context.h -- device + stream ownership and error checking.
//
// Mirrors AclContext / check_acl (src/csrc/include/minicpmv/acl_context.h:11-33):
// one device and one stream per context, every runtime error a
// std::runtime_error.  The stream is created at the default priority.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace minicpmv {

inline void check_hip(hipError_t code, const char* expr) {
    if (code != hipSuccess) {
        throw std::runtime_error(std::string(expr) + " failed with hipError=" + std::to_string(static_cast<int>(code)) +
                                 " (" + hipGetErrorString(code) + ")");
    }
}

// Throws std::runtime_error("<what> failed: <mcv_last_error()>") on a non-zero
// status from the C-ABI (include/mcv_quant.h).
void check_mcv(int status, const char* what);

// A u32 in host-mapped pinned memory (hipHostMalloc, mapped and coherent)
// that the kernels with bounded cross-workgroup waits set to 1 when a wait
// gives up.  The host reads it with a plain load -- no synchronisation, no
// copy -- so an operator object can check it at every call and at every
// point where its caller synchronises anyway.  Move-only.
class WaitStatus {
public:
    WaitStatus();
    ~WaitStatus();
    WaitStatus(WaitStatus&& other) noexcept;
    WaitStatus& operator=(WaitStatus&& other) noexcept;
    WaitStatus(const WaitStatus&) = delete;
    WaitStatus& operator=(const WaitStatus&) = delete;

    // The word's device address, for the C-ABI's `status` argument.
    uint32_t* device_word() const { return dev_; }
    bool gave_up() const;
    void clear();

private:
    uint32_t* host_{nullptr};
    uint32_t* dev_{nullptr};
};

class HipContext {
public:
    explicit HipContext(int device_id = 0);
    ~HipContext();

    HipContext(const HipContext&) = delete;
    HipContext& operator=(const HipContext&) = delete;

    int device_id() const { return device_id_; }
    hipStream_t stream() const { return stream_; }
    void synchronize() const;

private:
    int device_id_;
    hipStream_t stream_{nullptr};
};

}  // namespace minicpmv

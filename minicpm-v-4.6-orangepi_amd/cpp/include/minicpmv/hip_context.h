// hip_context.h -- device + stream ownership and error checking.
//
// Mirrors AclContext / check_acl (src/csrc/include/minicpmv/acl_context.h:11-33):
// one device and one stream per context, every runtime error a
// std::runtime_error.  The stream is created at the default priority.
#pragma once

#include <hip/hip_runtime_api.h>

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

// hip_context.cpp -- HipContext and C-ABI status checking.
#include "minicpmv/hip_context.h"

#include "mcv_quant.h"

#include <utility>

namespace minicpmv {

void check_mcv(int status, const char* what) {
    if (status != MCV_OK) {
        throw std::runtime_error(std::string(what) + " failed: " + mcv_last_error());
    }
}

WaitStatus::WaitStatus() {
    void* p = nullptr;
    check_hip(hipHostMalloc(&p, sizeof(uint32_t), hipHostMallocMapped | hipHostMallocCoherent), "hipHostMalloc");
    host_ = static_cast<uint32_t*>(p);
    *host_ = 0;
    void* d = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&d, p, 0);
    if (e != hipSuccess) {
        (void)hipHostFree(p);
        host_ = nullptr;
        check_hip(e, "hipHostGetDevicePointer");
    }
    dev_ = static_cast<uint32_t*>(d);
}

WaitStatus::~WaitStatus() {
    if (host_ != nullptr) (void)hipHostFree(host_);
}

WaitStatus::WaitStatus(WaitStatus&& other) noexcept
    : host_(std::exchange(other.host_, nullptr)), dev_(std::exchange(other.dev_, nullptr)) {}

WaitStatus& WaitStatus::operator=(WaitStatus&& other) noexcept {
    if (this != &other) {
        if (host_ != nullptr) (void)hipHostFree(host_);
        host_ = std::exchange(other.host_, nullptr);
        dev_ = std::exchange(other.dev_, nullptr);
    }
    return *this;
}

bool WaitStatus::gave_up() const {
    return host_ != nullptr && __atomic_load_n(host_, __ATOMIC_ACQUIRE) != 0;
}

void WaitStatus::clear() {
    if (host_ != nullptr) __atomic_store_n(host_, 0u, __ATOMIC_RELEASE);
}

HipContext::HipContext(int device_id) : device_id_(device_id) {
    check_hip(hipSetDevice(device_id_), "hipSetDevice");
    check_hip(hipStreamCreate(&stream_), "hipStreamCreate");
}

HipContext::~HipContext() {
    if (stream_ != nullptr) {
        (void)hipStreamSynchronize(stream_);
        (void)hipStreamDestroy(stream_);
    }
}

void HipContext::synchronize() const { check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize"); }

}  // namespace minicpmv

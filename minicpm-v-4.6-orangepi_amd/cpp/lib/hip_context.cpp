// hip_context.cpp -- HipContext and C-ABI status checking.
#include "minicpmv/hip_context.h"

#include "mcv_quant.h"

namespace minicpmv {

void check_mcv(int status, const char* what) {
    if (status != MCV_OK) {
        throw std::runtime_error(std::string(what) + " failed: " + mcv_last_error());
    }
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

// decode_dispatch.cpp -- W8A8 / W4A16 / dense choice per projection.
#include "minicpmv/decode_dispatch.h"

#include "minicpmv/ops.h"

#include <cstdlib>
#include <stdexcept>

namespace minicpmv {

bool w8a8_decode_enabled_for_layers() {
    static const bool enabled = [] {
        const char* v = std::getenv("MINICPM_W8A8_DECODE");
        return v != nullptr && std::string(v) != "0" && std::string(v) != "false";
    }();
    return enabled;
}

std::string w8a8_decode_mode() {
    static const std::string mode = [] {
        const char* v = std::getenv("MINICPM_W8A8_DECODE");
        return v == nullptr ? std::string{} : std::string(v);
    }();
    return mode;
}

bool w8a8_decode_enabled() {
    const std::string mode = w8a8_decode_mode();
    return !mode.empty() && mode != "0" && mode != "false";
}

bool w8a8_policy_allows(const char* token) {
    if (!w8a8_decode_enabled()) return false;
    const std::string mode = w8a8_decode_mode();
    if (mode == "all") return true;
    const std::string t(token);
    if (mode == "1" || mode == "selective") return t == "lm_head";
    return mode.find(t) != std::string::npos;
}

bool w8a8_weight_ready(const W8A8QuantizedWeight* w8_weight) {
    return w8a8_decode_enabled_for_layers() && w8_weight != nullptr && w8_weight->w_int8.data() != nullptr;
}

void matmul_decode_w8a8_prequant(const Tensor& x_int8, const Tensor& x_scale, const W8A8QuantizedWeight& w8_weight,
                                 Tensor& out, hipStream_t stream) {
    matmul_w8a8(x_int8, x_scale, w8_weight, out, stream);
}

void matmul_decode_dispatch(const Tensor& x, const Tensor* dense_weight, const W4A16QuantizedWeight* quant_weight,
                            const W8A8QuantizedWeight* w8_weight, Tensor& out, hipStream_t stream) {
    if (w8a8_weight_ready(w8_weight) && x.shape().size() == 2) {
        Tensor x_int8(x.shape(), DType::Int8);
        x_int8.allocate();
        Tensor x_scale({x.shape()[0]}, DType::Float32);
        x_scale.allocate();
        w8a8_quantize(x, x_int8, x_scale, stream);
        matmul_decode_w8a8_prequant(x_int8, x_scale, *w8_weight, out, stream);
        // The temporaries are freed on return; hipFree waits for the kernels.
        return;
    }
    if (quant_weight != nullptr && quant_weight->w_int8.data() != nullptr && x.shape().size() == 2) {
        matmul_w4a16(x, *quant_weight, out, stream);
        return;
    }
    if (dense_weight == nullptr) throw std::runtime_error("matmul_decode_dispatch: no weight for this projection");
    matmul_b_transposed(x, *dense_weight, out, stream);
}

}  // namespace minicpmv

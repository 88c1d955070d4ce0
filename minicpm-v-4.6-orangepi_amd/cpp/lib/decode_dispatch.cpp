// decode_dispatch.cpp -- W8A8 / W4A16 / dense choice per projection.
#include "minicpmv/decode_dispatch.h"

#include "minicpmv/hip_context.h"
#include "minicpmv/ops.h"

#include <cstdlib>
#include <stdexcept>
#include <map>
#include <utility>

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

void DecodeScratch::reserve(int64_t M, int64_t K) {
    if (static_cast<int64_t>(x_int8.numel()) < M * K) {
        x_int8 = Tensor({M * K}, DType::Int8);
        x_int8.allocate();
    }
    if (static_cast<int64_t>(x_scale.numel()) < M) {
        x_scale = Tensor({M}, DType::Float16);
        x_scale.allocate();
    }
}

namespace {

bool rank2(const Tensor& x) { return x.shape().size() == 2; }

void w8a8_branch(const Tensor& x, const W8A8QuantizedWeight& w8, Tensor& out, hipStream_t stream,
                 DecodeScratch& scratch) {
    const int64_t M = x.shape()[0], K = x.shape()[1];
    scratch.reserve(M, K);
    // Non-owning tensors of the operators' shapes over the scratch bytes.
    Tensor xq = Tensor::view(scratch.x_int8, {M, K}, DType::Int8);
    Tensor xs = Tensor::view(scratch.x_scale, {M}, DType::Float16);
    w8a8_quantize(x, xq, xs, stream);
    matmul_decode_w8a8_prequant(xq, xs, w8, out, stream);
}

}  // namespace

void matmul_decode_dispatch(const Tensor& x, const Tensor* dense_weight, const W4A16QuantizedWeight* quant_weight,
                            const W8A8QuantizedWeight* w8_weight, Tensor& out, hipStream_t stream,
                            DecodeScratch& scratch) {
    const bool one_row = rank2(x) && x.shape()[0] == 1;
    const bool q4_ready = quant_weight != nullptr && quant_weight->w_int8.data() != nullptr;
    if (w8a8_weight_ready(w8_weight) && one_row) {
        w8a8_branch(x, *w8_weight, out, stream, scratch);
        return;
    }
    if (q4_ready && one_row) {
        matmul_w4a16(x, *quant_weight, out, stream, scratch.gemm_ws);
        return;
    }
    if (dense_weight != nullptr) {
        matmul_b_transposed(x, *dense_weight, out, stream);
        return;
    }
    if (q4_ready && rank2(x)) {
        matmul_w4a16(x, *quant_weight, out, stream, scratch.gemm_ws);
        return;
    }
    if (w8a8_weight_ready(w8_weight) && rank2(x)) {
        w8a8_branch(x, *w8_weight, out, stream, scratch);
        return;
    }
    throw std::runtime_error("matmul_decode_dispatch: no weight for this projection");
}

void matmul_decode_dispatch(const Tensor& x, const Tensor* dense_weight, const W4A16QuantizedWeight* quant_weight,
                            const W8A8QuantizedWeight* w8_weight, Tensor& out, hipStream_t stream) {
    thread_local std::map<std::pair<int, hipStream_t>, DecodeScratch> per_stream;
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    matmul_decode_dispatch(x, dense_weight, quant_weight, w8_weight, out, stream, per_stream[{dev, stream}]);
}

}  // namespace minicpmv

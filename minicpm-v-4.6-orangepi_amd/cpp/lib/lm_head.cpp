// lm_head.cpp -- greedy lm_head over quantised vocabulary projections.
#include "minicpmv/lm_head.h"

#include "mcv_quant.h"
#include "minicpmv/hip_context.h"
#include "minicpmv/ops.h"

#include <stdexcept>

namespace minicpmv {

LmHeadW4A16 make_lm_head_w4a16(W4A16QuantizedWeight weight, int64_t vocab) {
    if (vocab <= 0 || vocab > weight.N) throw std::runtime_error("lm_head vocab must be in [1, weight N]");
    LmHeadW4A16 head;
    head.weight = std::move(weight);
    head.vocab = vocab;
    head.workspace = Tensor({mcv_lm_head_workspace_bytes(vocab)}, DType::UInt8);
    head.workspace.zero();
    head.token = Tensor({1}, DType::Int64);
    head.token.zero();
    head.slots = Tensor({mcv_lm_head_slots_bytes()}, DType::UInt8);
    head.slots.zero();
    return head;
}

void lm_head_argmax_w4a16(const Tensor& hidden_1xH, LmHeadW4A16& head, Tensor* logits, hipStream_t stream) {
    const W4A16QuantizedWeight& w = head.weight;
    if (hidden_1xH.dtype() != DType::Float16 || hidden_1xH.shape() != std::vector<int64_t>{1, w.K})
        throw std::runtime_error("lm_head hidden must be fp16 [1, hidden_size]");
    if (logits && (logits->dtype() != DType::Float16 || static_cast<int64_t>(logits->numel()) != head.vocab))
        throw std::runtime_error("lm_head logits must be fp16 [1, vocab]");
    check_mcv(mcv_w4a16_lm_head_argmax(hidden_1xH.data(), w.K, w.N, head.vocab, w.w_int8.data(), w.scales.data(),
                                       w.zeros.data(), w.zero_bias, logits ? logits->data() : nullptr,
                                       static_cast<int64_t*>(head.token.data()), head.workspace.data(), stream),
              "lm_head_argmax_w4a16");
}

uint32_t lm_head_argmax_slots_w4a16(const Tensor& hidden_1xH, LmHeadW4A16& head, Tensor* logits, hipStream_t stream) {
    const W4A16QuantizedWeight& w = head.weight;
    if (hidden_1xH.dtype() != DType::Float16 || hidden_1xH.shape() != std::vector<int64_t>{1, w.K})
        throw std::runtime_error("lm_head hidden must be fp16 [1, hidden_size]");
    if (logits && (logits->dtype() != DType::Float16 || static_cast<int64_t>(logits->numel()) != head.vocab))
        throw std::runtime_error("lm_head logits must be fp16 [1, vocab]");
    if (head.tag >= MCV_LM_SLOT_TAG_MAX) {          // tags must grow: start over from zero-filled slots
        check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
        head.slots.zero();
        head.tag = 0;
    }
    const uint32_t tag = ++head.tag;
    check_mcv(mcv_w4a16_lm_head_argmax_slots(hidden_1xH.data(), w.K, w.N, head.vocab, w.w_int8.data(),
                                             w.scales.data(), w.zeros.data(), w.zero_bias,
                                             logits ? logits->data() : nullptr, head.slots.data(), tag, stream),
              "lm_head_argmax_slots_w4a16");
    return tag;
}

int64_t lm_head_read_slots_token(const LmHeadW4A16& head, uint32_t tag, hipStream_t stream) {
    uint64_t host[MCV_LM_SLOTS * MCV_LM_SLOT_STRIDE];
    check_hip(hipMemcpyAsync(host, head.slots.data(), sizeof(host), hipMemcpyDeviceToHost, stream),
              "hipMemcpyAsync slots");
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    return mcv_lm_head_slots_token(host, tag);
}

namespace {

const Tensor& maybe_norm(const Tensor& hidden, const Tensor* final_norm, double eps, Tensor& normed,
                         hipStream_t stream) {
    if (final_norm == nullptr) return hidden;
    normed = Tensor(hidden.shape(), DType::Float16);
    normed.allocate();
    rms_norm(hidden, *final_norm, normed, eps, stream);
    return normed;
}

int64_t read_token(const Tensor& token, hipStream_t stream) {
    int64_t t = 0;
    check_hip(hipMemcpyAsync(&t, token.data(), sizeof(t), hipMemcpyDeviceToHost, stream), "hipMemcpyAsync token");
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    return t;
}

}  // namespace

int64_t lm_head_greedy_w4a16(const Tensor& last_hidden_1xH, const Tensor* final_norm, double rms_epsilon,
                             LmHeadW4A16& head, hipStream_t stream) {
    Tensor normed;
    const Tensor& x = maybe_norm(last_hidden_1xH, final_norm, rms_epsilon, normed, stream);
    const uint32_t tag = lm_head_argmax_slots_w4a16(x, head, nullptr, stream);
    return lm_head_read_slots_token(head, tag, stream);
}

int64_t lm_head_greedy_w8a8(const Tensor& last_hidden_1xH, const Tensor* final_norm, double rms_epsilon,
                            const W8A8QuantizedWeight& head, int64_t vocab, hipStream_t stream) {
    if (last_hidden_1xH.shape() != std::vector<int64_t>{1, head.K})
        throw std::runtime_error("lm_head hidden must be [1, hidden_size]");
    if (vocab <= 0 || vocab > head.N) throw std::runtime_error("lm_head vocab must be in [1, weight N]");
    Tensor normed;
    const Tensor& x = maybe_norm(last_hidden_1xH, final_norm, rms_epsilon, normed, stream);
    Tensor xq({1, head.K}, DType::Int8);
    xq.allocate();
    Tensor xs({1}, DType::Float32);
    xs.allocate();
    w8a8_quantize(x, xq, xs, stream);
    Tensor logits({1, head.N}, DType::Float16);
    logits.allocate();
    matmul_w8a8(xq, xs, head, logits, stream);
    Tensor token({1}, DType::Int64);
    token.allocate();
    check_mcv(mcv_argmax_f16(logits.data(), 1, vocab, static_cast<int64_t*>(token.data()), stream), "lm_head argmax");
    return read_token(token, stream);
}

}  // namespace minicpmv

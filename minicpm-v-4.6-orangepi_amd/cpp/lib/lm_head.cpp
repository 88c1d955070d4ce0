// lm_head.cpp -- greedy lm_head over quantised vocabulary projections.
#include "minicpmv/lm_head.h"

#include "mcv_quant.h"
#include "minicpmv/ops.h"

#include <stdexcept>

namespace minicpmv {

LmHeadW4A16 make_lm_head_w4a16(W4A16QuantizedWeight weight, int64_t vocab) {
    if (vocab <= 0 || vocab > weight.N) throw std::runtime_error("lm_head vocab must be in [1, weight N]");
    if (weight.dense_kn.numel() > 0)
        throw std::runtime_error("make_lm_head_w4a16: the weight is kept dense (GPTQ act-order blocks span more than "
                                 "16 levels); the lm_head takes slab-layout weights");
    LmHeadW4A16 head;
    head.weight = std::move(weight);
    head.vocab = vocab;
    head.workspace = Tensor({mcv_lm_head_workspace_bytes(vocab)}, DType::UInt8);
    head.workspace.zero();
    head.token = Tensor({1}, DType::Int64);
    head.token.zero();
    head.slots = Tensor({mcv_lm_head_slots_bytes()}, DType::UInt8);
    head.slots.zero();
    head.normed = Tensor({1, head.weight.K}, DType::Float16);
    head.normed.allocate();
    return head;
}

namespace {

void check_io(const Tensor& hidden_1xH, const LmHeadW4A16& head, const Tensor* logits) {
    const W4A16QuantizedWeight& w = head.weight;
    if (hidden_1xH.dtype() != DType::Float16 || hidden_1xH.shape() != std::vector<int64_t>{1, w.K})
        throw std::runtime_error("lm_head hidden must be fp16 [1, hidden_size]");
    if (logits && (logits->dtype() != DType::Float16 || static_cast<int64_t>(logits->numel()) != head.vocab))
        throw std::runtime_error("lm_head logits must be fp16 [1, vocab]");
}

// A give-up is reported once: the workspace (whose u32 at byte 0 holds the
// sticky give-up flag) is zero-filled after the stream drains and the status
// word cleared before the error is raised, so the next call reports only its
// own outcome.
[[noreturn]] void raise_gave_up(LmHeadW4A16& head, hipStream_t stream) {
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    head.workspace.zero();
    head.status.clear();
    throw std::runtime_error(
        "lm_head_argmax_w4a16: the wait for the workgroups' argmax keys gave up (token -1); the workspace was reset");
}

}  // namespace

void lm_head_argmax_w4a16(const Tensor& hidden_1xH, LmHeadW4A16& head, Tensor* logits, hipStream_t stream) {
    check_io(hidden_1xH, head, logits);
    if (head.status.gave_up()) raise_gave_up(head, stream);
    const W4A16QuantizedWeight& w = head.weight;
    check_mcv(mcv_w4a16_lm_head_argmax(hidden_1xH.data(), w.K, w.N, head.vocab, w.w_int8.data(), w.scales.data(),
                                       w.zeros.data(), w.zero_bias, logits ? logits->data() : nullptr,
                                       static_cast<int64_t*>(head.token.data()), head.workspace.data(),
                                       head.status.device_word(), stream),
              "lm_head_argmax_w4a16");
}

int64_t lm_head_read_token(LmHeadW4A16& head, hipStream_t stream) {
    int64_t t = 0;
    check_hip(hipMemcpyAsync(&t, head.token.data(), sizeof(t), hipMemcpyDeviceToHost, stream), "hipMemcpyAsync token");
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    if (t < 0 || head.status.gave_up()) raise_gave_up(head, stream);
    return t;
}

uint32_t lm_head_argmax_slots_w4a16(const Tensor& hidden_1xH, LmHeadW4A16& head, Tensor* logits, hipStream_t stream) {
    check_io(hidden_1xH, head, logits);
    const W4A16QuantizedWeight& w = head.weight;
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

int64_t lm_head_greedy_w4a16(const Tensor& last_hidden_1xH, const Tensor* final_norm, double rms_epsilon,
                             LmHeadW4A16& head, hipStream_t stream) {
    const Tensor* x = &last_hidden_1xH;
    if (final_norm != nullptr) {
        rms_norm(last_hidden_1xH, *final_norm, head.normed, rms_epsilon, stream);
        x = &head.normed;
    }
    const uint32_t tag = lm_head_argmax_slots_w4a16(*x, head, nullptr, stream);
    return lm_head_read_slots_token(head, tag, stream);
}

LmHeadW8A8 make_lm_head_w8a8(const W8A8QuantizedWeight& weight, int64_t vocab) {
    if (vocab <= 0 || vocab > weight.N) throw std::runtime_error("lm_head vocab must be in [1, weight N]");
    if (weight.w_int8.data() == nullptr || weight.w_scale.data() == nullptr)
        throw std::runtime_error("lm_head W8A8 weight is not loaded");
    LmHeadW8A8 head;
    head.weight = &weight;
    head.vocab = vocab;
    head.normed = Tensor({1, weight.K}, DType::Float16);
    head.xq = Tensor({1, weight.K}, DType::Int8);
    head.xs = Tensor({1}, DType::Float16);
    head.logits = Tensor({1, weight.N}, DType::Float16);
    head.keys = Tensor({(vocab + 63) / 64}, DType::Int64);
    head.token = Tensor({1}, DType::Int64);
    for (Tensor* t : {&head.normed, &head.xq, &head.xs, &head.logits, &head.keys, &head.token}) t->allocate();
    head.workspace = Tensor({mcv_lm_head_workspace_bytes(vocab)}, DType::UInt8);
    head.workspace.zero();
    return head;
}

int64_t lm_head_greedy_w8a8(const Tensor& last_hidden_1xH, const Tensor* final_norm, double rms_epsilon,
                            LmHeadW8A8& head, hipStream_t stream) {
    const W8A8QuantizedWeight& w = *head.weight;
    if (last_hidden_1xH.dtype() != DType::Float16 || last_hidden_1xH.shape() != std::vector<int64_t>{1, w.K})
        throw std::runtime_error("lm_head hidden must be fp16 [1, hidden_size]");
    const Tensor* x = &last_hidden_1xH;
    if (final_norm != nullptr) {
        rms_norm(last_hidden_1xH, *final_norm, head.normed, rms_epsilon, stream);
        x = &head.normed;
    }
    int64_t* token = static_cast<int64_t*>(head.token.data());
    if (w.layout == MCV_W8_TILED && w.K <= 2048) {
        // one launch: the activation quantisation with the fp16 x_scale (as
        // language_model.cpp:439-441), the GEMV with the fp16 w_scale (:465-466)
        // and the argmax on the device
        check_mcv(mcv_w8a8_lm_head_argmax(x->data(), w.K, w.N, head.vocab, static_cast<const int8_t*>(w.w_int8.data()),
                                          w.w_scale.data(), MCV_F16, MCV_F16, head.logits.data(), token,
                                          head.workspace.data(), nullptr, stream),
                  "lm_head W8A8");
    } else if (w.layout == MCV_W8_TILED) {
        // the same in three launches: quantisation, the GEMV with one argmax
        // key per slab, the keys' reduction
        w8a8_quantize(*x, head.xq, head.xs, stream);
        check_mcv(mcv_w8a8_gemv_argmax_partials(static_cast<const int8_t*>(head.xq.data()), head.xs.data(), MCV_F16,
                                                w.K, w.N, head.vocab, static_cast<const int8_t*>(w.w_int8.data()),
                                                w.w_scale.data(), MCV_F16, head.logits.data(), head.keys.data(),
                                                stream),
                  "lm_head W8A8 GEMV");
        check_mcv(mcv_argmax_reduce_keys(head.keys.data(), head.keys.numel(), token, stream), "lm_head argmax");
    } else {
        w8a8_quantize(*x, head.xq, head.xs, stream);
        matmul_w8a8(head.xq, head.xs, w, head.logits, stream);
        check_mcv(mcv_argmax_f16(head.logits.data(), 1, head.vocab, token, stream), "lm_head argmax");
    }
    int64_t t = 0;
    check_hip(hipMemcpyAsync(&t, head.token.data(), sizeof(t), hipMemcpyDeviceToHost, stream), "hipMemcpyAsync token");
    check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
    if (t < 0) {
        // the bounded wait for the workgroups' keys gave up: reset the
        // workspace's give-up word and report it
        head.workspace.zero();
        throw std::runtime_error("lm_head_greedy_w8a8: the wait for the workgroups' argmax keys gave up (token -1)");
    }
    return t;
}

}  // namespace minicpmv

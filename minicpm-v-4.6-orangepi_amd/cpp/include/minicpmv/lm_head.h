// lm_head.h -- greedy lm_head over a W4A16 (or W8A8) vocabulary projection.
//
// Replaces lm_head_greedy (src/csrc/lib/language_model.cpp:412-482): final
// RMSNorm, then -- instead of 16 chunk matmuls, 16 blocking D2H copies and a
// host scan -- one GEMV with the argmax folded into it.  Same tie rule: the
// first maximum wins, fp16 subnormals compare as zero, NaN never wins.
#pragma once

#include "minicpmv/quantized_weight.h"
#include "minicpmv/tensor.h"

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace minicpmv {

struct LmHeadW4A16 {
    W4A16QuantizedWeight weight;   // [hidden, >= vocab]
    int64_t vocab{0};
    Tensor workspace;              // zero-filled once; calls keep its counters and tagged keys consistent
    Tensor token;                  // Int64 [1]
    Tensor slots;                  // tagged slot maxima of the host-finished argmax
    uint32_t tag{0};               // tag of the last slots call
};

LmHeadW4A16 make_lm_head_w4a16(W4A16QuantizedWeight weight, int64_t vocab);

// Stream-ordered: token and (optional, fp16 [1, vocab]) logits on the device.
void lm_head_argmax_w4a16(const Tensor& hidden_1xH, LmHeadW4A16& head, Tensor* logits, hipStream_t stream);

// Stream-ordered, host-finished argmax: the GEMV leaves call-tagged maxima in
// head.slots (no device round trip at the end of the kernel); returns the tag
// to pass to lm_head_read_slots_token.
uint32_t lm_head_argmax_slots_w4a16(const Tensor& hidden_1xH, LmHeadW4A16& head, Tensor* logits, hipStream_t stream);
// Copies the slots to the host (synchronises `stream`) and folds them into the token.
int64_t lm_head_read_slots_token(const LmHeadW4A16& head, uint32_t tag, hipStream_t stream);

// lm_head_greedy semantics: optional final RMSNorm (final_norm may be null),
// then the argmax through the slots; returns the token on the host
// (synchronises `stream`).
int64_t lm_head_greedy_w4a16(const Tensor& last_hidden_1xH, const Tensor* final_norm, double rms_epsilon,
                             LmHeadW4A16& head, hipStream_t stream);

// W8A8 variant (language_model.cpp:434-467): one activation quantisation, the
// fused int8 GEMM over [hidden, vocab], argmax on the device.
int64_t lm_head_greedy_w8a8(const Tensor& last_hidden_1xH, const Tensor* final_norm, double rms_epsilon,
                            const W8A8QuantizedWeight& head, int64_t vocab, hipStream_t stream);

}  // namespace minicpmv
